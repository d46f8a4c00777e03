"""The C ABI without a GPU: the built library loads and exports every function
include/dan_tree_attn.h, dan_qkv_front.h, dan_tree_plan.h, dan_fp8.h and dan_gdn.h declare, the ctypes mirror has the header's exact
struct layout (checked by compiling the header with gcc), and argument
errors come back as status codes with messages before any GPU call."""
import ctypes
import os
import re
import subprocess

import pytest

from dan_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dan_tree_attn.h")
FRONT_HEADER = os.path.join(ROOT, "include", "dan_qkv_front.h")
PLAN_HEADER = os.path.join(ROOT, "include", "dan_tree_plan.h")
FP8_HEADER = os.path.join(ROOT, "include", "dan_fp8.h")
GDN_HEADER = os.path.join(ROOT, "include", "dan_gdn.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_native.LIB_PATH):
        from dan_amd import _build

        _build.build()
    return _native.load()


def declared_functions():
    text = "".join(open(h).read() for h in (HEADER, FRONT_HEADER, PLAN_HEADER, FP8_HEADER, GDN_HEADER))
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(dan_\w+)\s*\(", text, re.M)))


def test_exports_every_declared_function(lib):
    names = declared_functions()
    assert set(names) == set(_native.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (dan_\w+)", out))
    assert set(names) <= exported


STRUCTS = {
    "DanUnit": _native.DanUnit,
    "DanSegmentDesc": _native.DanSegmentDesc,
    "DanPastDesc": _native.DanPastDesc,
    "DanWorkItem": _native.DanWorkItem,
    "DanTreeAttnArgs": _native.DanTreeAttnArgs,
    "DanFrontSave": _native.DanFrontSave,
    "DanQkvFrontArgs": _native.DanQkvFrontArgs,
    "DanTreePlanArgs": _native.DanTreePlanArgs,
    "DanFp8QuantArgs": _native.DanFp8QuantArgs,
    "DanFp8GemmArgs": _native.DanFp8GemmArgs,
    "DanGdnArgs": _native.DanGdnArgs,
    "DanGdnConvArgs": _native.DanGdnConvArgs,
}


def test_ctypes_layout_matches_header(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "dan_tree_attn.h"', '#include "dan_qkv_front.h"',
             '#include "dan_tree_plan.h"', '#include "dan_fp8.h"', '#include "dan_gdn.h"', "int main(void) {"]
    for cname, cls in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append(f'printf("ABI %d\\n", DAN_TREE_ATTN_ABI_VERSION);')
    lines.append(f'printf("KEY_TILE %d\\n", DAN_TREE_ATTN_KEY_TILE);')
    lines.append('printf("SCRATCH %lld\\n", (long long)DAN_TREE_ATTN_SCRATCH_BYTES);')
    lines.append('printf("PHASES %d,%d,%d\\n", DAN_TREE_ATTN_PHASES_ALL, DAN_TREE_ATTN_PHASE_PACK, DAN_TREE_ATTN_PHASE_ATTEND);')
    lines.append('printf("FRONT %d,%d,%d,%d\\n", DAN_QKV_FRONT_ABI_VERSION, DAN_FRONT_NORM_NONE, DAN_FRONT_NORM_RMS, '
                 'DAN_FRONT_NORM_RMS_ZERO_CENTERED);')
    lines.append('printf("PLAN %d,%d,%d,%d,%d\\n", DAN_TREE_PLAN_ABI_VERSION, DAN_TREE_PLAN_MAX_WORK, '
                 'DAN_TREE_PLAN_MAX_SLOTS, DAN_TREE_PLAN_MAX_SEGMENTS, DAN_TREE_PLAN_MAX_BRANCHES);')
    lines.append('printf("FP8 %d,%d,%d,%d,%d,%d,%d,%d,%d\\n", DAN_FP8_ABI_VERSION, DAN_FP8_SCALE_TENSOR, DAN_FP8_SCALE_ROW, '
                 'DAN_FP8_GEMM_X_SCALE_TENSOR, DAN_FP8_GEMM_W_SCALE_TENSOR, DAN_FP8_GEMM_X_TILED, DAN_FP8_GEMM_W_TILED, '
                 'DAN_FP8_LAYOUT_ROWS, DAN_FP8_LAYOUT_TILED);')
    lines.append('printf("GDN %d\\n", DAN_GDN_ABI_VERSION);')
    lines.append("return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                               check=True).stdout.splitlines())
    for cname, cls in STRUCTS.items():
        assert int(got[f"{cname} size"]) == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(cls, fname).offset, f"{cname}.{fname}"
    assert int(got["ABI"]) == _native.ABI_VERSION
    assert int(got["KEY_TILE"]) == _native.KEY_TILE
    assert int(got["SCRATCH"]) == _native.SCRATCH_BYTES
    assert got["PHASES"] == f"{_native.PHASES_ALL},{_native.PHASE_PACK},{_native.PHASE_ATTEND}"
    assert got["FRONT"] == (f"{_native.FRONT_ABI_VERSION},{_native.FRONT_NORM_NONE},{_native.FRONT_NORM_RMS},"
                            f"{_native.FRONT_NORM_RMS_ZERO_CENTERED}")
    assert got["FP8"] == (f"{_native.FP8_ABI_VERSION},{_native.FP8_SCALE_TENSOR},{_native.FP8_SCALE_ROW},"
                          f"{_native.FP8_GEMM_X_SCALE_TENSOR},{_native.FP8_GEMM_W_SCALE_TENSOR},"
                          f"{_native.FP8_GEMM_X_TILED},{_native.FP8_GEMM_W_TILED},"
                          f"{_native.FP8_LAYOUT_ROWS},{_native.FP8_LAYOUT_TILED}")
    assert int(got["GDN"]) == _native.GDN_ABI_VERSION
    assert got["PLAN"] == (f"{_native.PLAN_ABI_VERSION},{_native.PLAN_MAX_WORK},{_native.PLAN_MAX_SLOTS},"
                           f"{_native.PLAN_MAX_SEGMENTS},{_native.PLAN_MAX_BRANCHES}")


def test_abi_version_and_tile_q(lib):
    assert lib.dan_tree_attn_abi_version() == _native.ABI_VERSION
    assert _native.tile_q(32, 8, 128, lib=lib) == 64   # rep 4: 4 heads x 64 tokens per work group
    assert _native.tile_q(8, 2, 128, lib=lib) == 64
    assert _native.tile_q(14, 2, 128, lib=lib) == 64   # rep 7: two head chunks
    assert _native.tile_q(16, 8, 128, lib=lib) == 128  # rep 2
    assert _native.tile_q(8, 8, 128, lib=lib) == 256   # rep 1
    assert _native.tile_q(8, 8, 64, lib=lib) == 256
    assert _native.tile_q(16, 2, 256, lib=lib) == 32   # head_dim 256: 4 waves, 4 heads x 32 tokens
    assert _native.tile_q(16, 8, 256, lib=lib) == 64
    assert _native.tile_q(8, 8, 256, lib=lib) == 128
    assert _native.tile_q(8, 8, 96, lib=lib) == 0      # head_dim not built
    assert _native.tile_q(12, 8, 128, lib=lib) == 0    # not a multiple
    assert _native.tile_q(0, 8, 128, lib=lib) == 0
    assert _native.head_groups(32, 8, lib) == 8     # rep 4: one chunk per kv head
    assert _native.head_groups(14, 2, lib) == 4     # rep 7: two chunks
    assert _native.head_groups(16, 8, lib) == 8
    assert _native.head_groups(12, 8, lib) == 0


def _args(**kw):
    a = _native.DanTreeAttnArgs()
    a.abi_version = _native.ABI_VERSION
    a.in_dtype = a.out_dtype = a.v_dtype = _native.DTYPE_BF16
    a.num_heads, a.num_kv_heads, a.head_dim, a.num_tokens = 32, 8, 128, 16
    a.scale = 0.088
    a.tile_q = 64
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,status,needle", [
    (dict(abi_version=99), _native.ERR_VERSION, "abi_version"),
    (dict(num_heads=30), _native.ERR_INVALID_ARGUMENT, "multiple"),
    (dict(head_dim=96), _native.ERR_UNSUPPORTED, "head_dim"),
    (dict(tile_q=32), _native.ERR_INVALID_ARGUMENT, "tile_q"),
    (dict(num_work=3), _native.ERR_INVALID_ARGUMENT, "NULL"),
    (dict(num_work=-1), _native.ERR_INVALID_ARGUMENT, "negative"),
    (dict(in_dtype=_native.DTYPE_E4M3, v_dtype=_native.DTYPE_E4M3, out_dtype=_native.DTYPE_F16),
     _native.ERR_UNSUPPORTED, "dtype"),
])
def test_argument_errors(lib, kw, status, needle):
    rc = lib.dan_tree_attn_fwd(ctypes.byref(_args(**kw)), None)
    assert rc == status
    assert needle in _native.last_error(lib)


def test_null_args(lib):
    assert lib.dan_tree_attn_fwd(None, None) == _native.ERR_INVALID_ARGUMENT
    assert "NULL" in _native.last_error(lib)


def test_empty_work_is_a_no_op(lib):
    """Nothing to do: success without touching the GPU."""
    assert lib.dan_tree_attn_fwd(ctypes.byref(_args(num_work=0)), None) == _native.OK
    assert _native.last_error(lib) == ""


def test_workspace_size(lib):
    # fp16 V^T, then one int32 exponent per (kv head, 64-column block), rounded up to 256 bytes
    assert _native.workspace_size(8, 128, 640, lib) == 8 * 128 * 640 * 2 + 512
    assert _native.workspace_size(1, 64, 64, lib) == 64 * 64 * 2 + 256
    assert _native.workspace_size(8, 128, 100, lib) == 0  # not a multiple of the key tile
    assert _native.workspace_size(0, 128, 64, lib) == 0


def test_bad_scale_dtype_and_workspace(lib):
    x = (ctypes.c_uint8 * 4096)()
    p = (ctypes.addressof(x) + 255) // 256 * 256
    full = dict(num_work=1, q=p, k=p, v=p, out=p, segments=p, work=p, key_lo=p, col_seg=p, vt_cols=64,
                workspace=p, workspace_bytes=8 * 128 * 64 * 2 + 256)
    # non-positive, infinite and NaN scales (checked from the float's bits: the
    # library is built with -fno-honor-nans, which may fold a NaN comparison)
    for bad_scale in (0.0, -0.0, -1.0, float("inf"), float("nan"), -float("nan")):
        assert lib.dan_tree_attn_fwd(ctypes.byref(_args(scale=bad_scale, **full)), None) == _native.ERR_INVALID_ARGUMENT
        assert "scale" in _native.last_error(lib)
    # 16-byte rows: misaligned pointers and strides are refused before launch
    for mis in (dict(q=p + 2), dict(out=p + 8), dict(k_stride_tok=1028), dict(v_stride_head=4)):
        assert lib.dan_tree_attn_fwd(ctypes.byref(_args(**dict(full, **mis))), None) == _native.ERR_INVALID_ARGUMENT
        assert "16-byte" in _native.last_error(lib)
    small = dict(full, workspace_bytes=100)
    assert lib.dan_tree_attn_fwd(ctypes.byref(_args(**small)), None) == _native.ERR_INVALID_ARGUMENT
    assert "workspace" in _native.last_error(lib)
    odd = dict(full, vt_cols=100)
    assert lib.dan_tree_attn_fwd(ctypes.byref(_args(**odd)), None) == _native.ERR_INVALID_ARGUMENT
    bad = _args(**dict(full, v_dtype=_native.DTYPE_E4M3))
    assert lib.dan_tree_attn_fwd(ctypes.byref(bad), None) == _native.ERR_UNSUPPORTED
    f8 = _args(**dict(full, in_dtype=_native.DTYPE_E4M3, v_dtype=_native.DTYPE_E4M3))  # no scales
    assert lib.dan_tree_attn_fwd(ctypes.byref(f8), None) == _native.ERR_INVALID_ARGUMENT
    assert "scale" in _native.last_error(lib)
    ph = _args(**dict(full, phases=3))
    assert lib.dan_tree_attn_fwd(ctypes.byref(ph), None) == _native.ERR_INVALID_ARGUMENT
    assert "phases" in _native.last_error(lib)
    # the attention launch needs a schedule of 1..units slots (1 item x 8 head groups here)
    for sched in (dict(), dict(units=p, sched_off=p, num_slots=0), dict(units=p, sched_off=p, num_slots=9),
                  dict(units=p, num_slots=8)):
        rc = lib.dan_tree_attn_fwd(ctypes.byref(_args(**dict(full, **sched))), None)
        assert rc == _native.ERR_INVALID_ARGUMENT
        assert "schedule" in _native.last_error(lib)


def test_noalloc_checks_before_any_gpu_call(lib):
    """dan_tree_attn_fwd_noalloc: NULL, version and a V^T copy larger than the
    library's scratch come back as status codes without a GPU; no work is a
    no-op."""
    assert lib.dan_tree_attn_fwd_noalloc(None, None) == _native.ERR_INVALID_ARGUMENT
    assert lib.dan_tree_attn_fwd_noalloc(ctypes.byref(_args(abi_version=3, num_work=1)), None) == _native.ERR_VERSION
    assert lib.dan_tree_attn_fwd_noalloc(ctypes.byref(_args(num_work=0)), None) == _native.OK
    cols = _native.SCRATCH_BYTES // (8 * 128 * 2) + 64  # one column block more than fits
    big = _args(num_work=1, vt_cols=cols)
    assert lib.dan_tree_attn_fwd_noalloc(ctypes.byref(big), None) == _native.ERR_UNSUPPORTED
    assert "scratch" in _native.last_error(lib)


def _front_args(**kw):
    a = _native.DanQkvFrontArgs()
    a.abi_version = _native.FRONT_ABI_VERSION
    a.dtype = _native.DTYPE_BF16
    a.num_tokens, a.num_heads, a.num_kv_heads, a.head_dim, a.rotary_dim = 4, 4, 2, 128, 128
    a.eps = 1e-6
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,status,needle", [
    (dict(abi_version=7), _native.ERR_VERSION, "abi_version"),
    (dict(head_dim=96), _native.ERR_UNSUPPORTED, "head_dim"),
    (dict(dtype=_native.DTYPE_F32), _native.ERR_UNSUPPORTED, "dtype"),
    (dict(rotary_dim=40), _native.ERR_INVALID_ARGUMENT, "rotary_dim"),
    (dict(rotary_dim=144), _native.ERR_INVALID_ARGUMENT, "rotary_dim"),
    (dict(norm=5), _native.ERR_INVALID_ARGUMENT, "norm"),
    (dict(norm=1), _native.ERR_INVALID_ARGUMENT, "weight"),
    (dict(num_saves=2), _native.ERR_INVALID_ARGUMENT, "saves"),
    (dict(num_heads=0), _native.ERR_INVALID_ARGUMENT, "head"),
])
def test_front_argument_errors(lib, kw, status, needle):
    assert lib.dan_qkv_front(ctypes.byref(_front_args(**kw)), None) == status
    assert needle in _native.last_error(lib)


def test_front_checks_pointers_and_alignment(lib):
    assert lib.dan_qkv_front(ctypes.byref(_front_args(num_tokens=0)), None) == _native.OK  # nothing to do
    x = (ctypes.c_uint8 * 8192)()
    p = (ctypes.addressof(x) + 255) // 256 * 256
    full = dict(q=p, k=p, v=p, cos=p, sin=p, q_out=p, k_out=p, q_stride_tok=512, q_stride_head=128, k_stride_tok=256,
                k_stride_head=128, qo_stride_tok=512, qo_stride_head=128, ko_stride_tok=256, ko_stride_head=128,
                cs_stride_tok=128)
    assert lib.dan_qkv_front(ctypes.byref(_front_args(**dict(full, q=0))), None) == _native.ERR_INVALID_ARGUMENT
    assert "NULL" in _native.last_error(lib)
    assert lib.dan_qkv_front(ctypes.byref(_front_args(**dict(full, q=p + 2))), None) == _native.ERR_INVALID_ARGUMENT
    assert "aligned" in _native.last_error(lib)
    assert lib.dan_qkv_front(ctypes.byref(_front_args(**dict(full, q_stride_tok=500))), None) == _native.ERR_INVALID_ARGUMENT
    assert "multiples of 8" in _native.last_error(lib)
    assert lib.dan_qkv_front(ctypes.byref(_front_args(**dict(full, cs_stride_tok=64))), None) == _native.ERR_INVALID_ARGUMENT
    assert "cs_stride_tok" in _native.last_error(lib)
    # a norm with a NaN, infinite or negative eps is refused (decided from the float's bits)
    normed = dict(full, norm=_native.FRONT_NORM_RMS, q_norm_weight=p, k_norm_weight=p)
    for bad_eps in (float("nan"), float("inf"), -1e-6):
        assert lib.dan_qkv_front(ctypes.byref(_front_args(**dict(normed, eps=bad_eps))), None) == _native.ERR_INVALID_ARGUMENT
        assert "eps" in _native.last_error(lib)


def test_plan_slots(lib):
    """k = max(1, min(num_cus // groups, num_work)) slots per head group, as
    dan_amd.plan.schedule makes them."""
    assert _native.plan_slots(130, 8, 256, lib) == 256
    assert _native.plan_slots(6, 8, 256, lib) == 48
    assert _native.plan_slots(5, 300, 256, lib) == 300
    assert _native.plan_slots(0, 8, 256, lib) == 0
    assert lib.dan_tree_attn_plan_abi_version() == _native.PLAN_ABI_VERSION


def _plan_args(**kw):
    a = _native.DanTreePlanArgs()
    a.abi_version = _native.PLAN_ABI_VERSION
    a.num_tokens, a.num_segments, a.num_branches, a.num_work, a.num_cols = 64, 1, 0, 1, 1
    a.tile_q, a.groups, a.num_cus, a.overhead = 64, 8, 256, 1
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,status,needle", [
    (dict(abi_version=7), _native.ERR_VERSION, "abi_version"),
    (dict(num_work=-1), _native.ERR_INVALID_ARGUMENT, "negative"),
    (dict(num_segments=0), _native.ERR_INVALID_ARGUMENT, "segments"),
    (dict(tile_q=0), _native.ERR_INVALID_ARGUMENT, "positive"),
    (dict(num_work=_native.PLAN_MAX_WORK + 1), _native.ERR_UNSUPPORTED, "num_work"),
    (dict(num_segments=_native.PLAN_MAX_SEGMENTS + 1), _native.ERR_UNSUPPORTED, "segments"),
    (dict(num_branches=_native.PLAN_MAX_BRANCHES + 1), _native.ERR_UNSUPPORTED, "branches"),
    (dict(groups=1, num_cus=1024), _native.ERR_INVALID_ARGUMENT, "NULL"),  # one slot (W = 1) but no tables
    (dict(), _native.ERR_INVALID_ARGUMENT, "NULL"),
])
def test_plan_argument_errors(lib, kw, status, needle):
    rc = lib.dan_tree_attn_plan(ctypes.byref(_plan_args(**kw)), None)
    assert rc == status
    assert needle in _native.last_error(lib)


def test_plan_too_many_slots(lib):
    a = _plan_args(num_work=1000, groups=1, num_cus=1024)
    assert lib.dan_tree_attn_plan(ctypes.byref(a), None) == _native.ERR_UNSUPPORTED
    assert "slots" in _native.last_error(lib)


def test_plan_empty_and_null(lib):
    assert lib.dan_tree_attn_plan(None, None) == _native.ERR_INVALID_ARGUMENT
    assert lib.dan_tree_attn_plan(ctypes.byref(_plan_args(num_work=0)), None) == _native.OK
    assert _native.last_error(lib) == ""


def _fp8_args(**kw):
    a = _native.DanFp8QuantArgs()
    a.abi_version = _native.FP8_ABI_VERSION
    a.dtype, a.rows, a.cols, a.mode, a.x_stride = _native.DTYPE_BF16, 4, 32, _native.FP8_SCALE_ROW, 32
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,status,needle", [
    (dict(abi_version=3), _native.ERR_VERSION, "abi_version"),
    (dict(dtype=_native.DTYPE_E4M3), _native.ERR_UNSUPPORTED, "dtype"),
    (dict(mode=5), _native.ERR_INVALID_ARGUMENT, "mode"),
    (dict(cols=24), _native.ERR_INVALID_ARGUMENT, "multiple of 16"),
    (dict(rows=-1), _native.ERR_INVALID_ARGUMENT, "negative"),
    (dict(rows=0, mode=_native.FP8_SCALE_TENSOR), _native.ERR_INVALID_ARGUMENT, "empty"),
    (dict(), _native.ERR_INVALID_ARGUMENT, "NULL"),
    (dict(x=16, xq=16, scale=16, x_stride=8), _native.ERR_INVALID_ARGUMENT, "aligned"),
])
def test_fp8_argument_errors(lib, kw, status, needle):
    rc = lib.dan_fp8_quantize(ctypes.byref(_fp8_args(**kw)), None)
    assert rc == status
    assert needle in _native.last_error(lib)


def test_fp8_empty_rows_is_a_no_op(lib):
    assert lib.dan_fp8_quantize(ctypes.byref(_fp8_args(rows=0)), None) == _native.OK
    assert lib.dan_fp8_abi_version() == _native.FP8_ABI_VERSION


def _gdn_args(**kw):
    a = _native.DanGdnArgs()
    a.abi_version = _native.GDN_ABI_VERSION
    a.dtype, a.num_k_heads, a.num_v_heads, a.k_dim, a.v_dim, a.num_runs = _native.DTYPE_BF16, 2, 4, 128, 128, 1
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,status,needle", [
    (dict(abi_version=9), _native.ERR_VERSION, "abi_version"),
    (dict(dtype=_native.DTYPE_F32), _native.ERR_UNSUPPORTED, "dtype"),
    (dict(k_dim=64), _native.ERR_UNSUPPORTED, "k_dim"),
    (dict(v_dim=36), _native.ERR_UNSUPPORTED, "v_dim"),
    (dict(num_v_heads=3), _native.ERR_INVALID_ARGUMENT, "multiple"),
    (dict(num_runs=-2), _native.ERR_INVALID_ARGUMENT, "negative"),
    (dict(), _native.ERR_INVALID_ARGUMENT, "NULL"),
])
def test_gdn_argument_errors(lib, kw, status, needle):
    rc = lib.dan_gdn_fwd(ctypes.byref(_gdn_args(**kw)), None)
    assert rc == status
    assert needle in _native.last_error(lib)


def _gdn_ptrs(**kw):
    # non-NULL, 16-byte aligned stand-ins: every case below fails its check before any launch
    ptrs = {f: 4096 for f in ("cu", "q", "k", "v", "g", "beta", "states_in", "states_out", "out", "workspace")}
    return _gdn_args(num_tokens=128, q_stride_tok=256, q_stride_head=128, k_stride_tok=256, k_stride_head=128,
                     **{**ptrs, **kw})


@pytest.mark.parametrize("kw,status,needle", [
    (dict(form=2), _native.ERR_INVALID_ARGUMENT, "form"),
    (dict(form=_native.GDN_FORM_CHUNK, v_dim=40), _native.ERR_UNSUPPORTED, "multiple of 32"),
    (dict(form=_native.GDN_FORM_CHUNK, workspace_bytes=4096), _native.ERR_INVALID_ARGUMENT, "workspace needs"),
    (dict(form=_native.GDN_FORM_TOKEN, workspace_bytes=1024), _native.ERR_INVALID_ARGUMENT, "workspace needs"),
    (dict(form=_native.GDN_FORM_CHUNK, state_index=4096, num_states_in=0), _native.ERR_INVALID_ARGUMENT,
     "num_states_in"),
])
def test_gdn_form_and_workspace_errors(lib, kw, status, needle):
    rc = lib.dan_gdn_fwd(ctypes.byref(_gdn_ptrs(**kw)), None)
    assert rc == status
    assert needle in _native.last_error(lib)


def test_gdn_workspace_size(lib):
    norms = (1000 * 2 * 2 * 4 + 255) // 256 * 256
    assert lib.dan_gdn_workspace_size(_native.GDN_FORM_TOKEN, 1000, 3, 2, 4, 128) == norms
    # chunk records: (runs + tokens // 64) slots x value heads x (T and A as bf16 pairs, 64 x 64 each,
    # K^T 128 x 64 bf16, five rows of 64 floats); the fp16 layout (T, A in fp32) fits in the same
    rec = (3 + 1000 // 64) * 4 * ((4 * 64 * 64 * 2 + 128 * 64 * 2) // 4 + 5 * 64) * 4
    assert lib.dan_gdn_workspace_size(_native.GDN_FORM_CHUNK, 1000, 3, 2, 4, 128) == rec
    assert lib.dan_gdn_workspace_size(7, 1000, 3, 2, 4, 128) == 0
    assert lib.dan_gdn_workspace_size(_native.GDN_FORM_CHUNK, -1, 3, 2, 4, 128) == 0


def test_gdn_no_runs_is_a_no_op(lib):
    assert lib.dan_gdn_fwd(ctypes.byref(_gdn_args(num_runs=0)), None) == _native.OK
    assert lib.dan_gdn_abi_version() == _native.GDN_ABI_VERSION


def _conv_args(**kw):
    a = _native.DanGdnConvArgs()
    a.abi_version = _native.GDN_ABI_VERSION
    a.dtype, a.channels, a.kernel, a.num_rows, a.num_ext, a.num_out = _native.DTYPE_BF16, 64, 4, 8, 11, 8
    a.src_stride, a.out_stride = 64, 64
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,status,needle", [
    (dict(abi_version=1), _native.ERR_VERSION, "abi_version"),
    (dict(dtype=_native.DTYPE_F32), _native.ERR_UNSUPPORTED, "dtype"),
    (dict(kernel=5), _native.ERR_UNSUPPORTED, "kernel"),
    (dict(channels=36), _native.ERR_UNSUPPORTED, "channels"),
    (dict(num_ext=-1), _native.ERR_INVALID_ARGUMENT, "negative"),
    (dict(), _native.ERR_INVALID_ARGUMENT, "NULL"),
    (dict(src=4096, ext=4096, take=4096, weight=4098, out=8192), _native.ERR_INVALID_ARGUMENT, "weight must be"),
])
def test_gdn_conv_argument_errors(lib, kw, status, needle):
    rc = lib.dan_gdn_conv(ctypes.byref(_conv_args(**kw)), None)
    assert rc == status
    assert needle in _native.last_error(lib)


def test_gdn_conv_no_rows_is_a_no_op(lib):
    assert lib.dan_gdn_conv(ctypes.byref(_conv_args(num_out=0)), None) == _native.OK


def test_stage_f16_checks_before_any_gpu_call(lib):
    """dan_tree_attn_stage_f16 (fp32 q / k -> fp16 with a power-of-2 scale):
    NULL, version, shape and alignment errors come back as status codes."""
    x = (ctypes.c_uint8 * 4096)()
    p = (ctypes.addressof(x) + 255) // 256 * 256

    def stage(**kw):
        a = _native.DanStageF16Args()
        a.abi_version = _native.ABI_VERSION
        a.d0, a.d1, a.d2 = 2, 3, 8
        a.x, a.stride0, a.stride1, a.out, a.scale, a.partial = p, 24, 8, p, p, p
        for k, v in kw.items():
            setattr(a, k, v)
        return lib.dan_tree_attn_stage_f16(ctypes.byref(a), None)

    assert lib.dan_tree_attn_stage_f16(None, None) == _native.ERR_INVALID_ARGUMENT
    assert stage(abi_version=5) == _native.ERR_VERSION
    assert stage(d2=6) == _native.ERR_INVALID_ARGUMENT and "multiple of 4" in _native.last_error(lib)
    assert stage(d0=-1) == _native.ERR_INVALID_ARGUMENT
    assert stage(scale=None) == _native.ERR_INVALID_ARGUMENT and "NULL" in _native.last_error(lib)
    for bad in (dict(x=p + 4), dict(stride1=6), dict(out=p + 2)):
        assert stage(**bad) == _native.ERR_INVALID_ARGUMENT and "aligned" in _native.last_error(lib)
