"""ctypes binding of the C ABI in include/dan_tree_attn.h (with
include/dan_qkv_front.h, include/dan_tree_plan.h, include/dan_fp8.h and
include/dan_gdn.h).

The shared library is plain C ABI (no torch types), built in-tree by
``dan_amd._build`` into ``dan_amd/_lib/``. It must be loaded after torch has
initialised its HIP runtime: torch's bundled ``libamdhip64.so`` carries the
soname the library links against, so both share one runtime and torch's
stream handles are valid in it.

There is no fallback: if the library is missing or cannot be loaded, every
entry point raises.
"""
import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "_lib")
LIB_NAME = "libdan_tree_attn.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

ABI_VERSION = 8
KEY_TILE = 64
SCRATCH_BYTES = 32 << 20  # DAN_TREE_ATTN_SCRATCH_BYTES: dan_tree_attn_fwd_noalloc's V^T scratch per GPU

# DanStatus
OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_LAUNCH, ERR_VERSION = range(5)
# DanDtype
DTYPE_BF16, DTYPE_F16, DTYPE_F32, DTYPE_E4M3 = range(4)
PHASES_ALL, PHASE_PACK, PHASE_ATTEND = 0, 1, 2

_i32, _i64, _f32, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class DanSegmentDesc(ctypes.Structure):
    _fields_ = [("start", _i32), ("n", _i32), ("trunk", _i32), ("past_len", _i32), ("past_idx", _i32),
                ("vt_col", _i32), ("reserved", _i32 * 2)]


class DanPastDesc(ctypes.Structure):
    _fields_ = [("k", _vp), ("v", _vp),
                ("k_stride_head", _i64), ("k_stride_tok", _i64),
                ("v_stride_head", _i64), ("v_stride_tok", _i64),
                ("k_scale", _vp), ("v_scale", _vp),
                ("len", _i32), ("reserved", _i32)]


class DanWorkItem(ctypes.Structure):
    _fields_ = [("seg", _i32), ("t0", _i32), ("tq", _i32), ("ja1", _i32), ("jb0", _i32), ("jb1", _i32),
                ("jfull", _i32), ("lo_max", _i32)]


class DanUnit(ctypes.Structure):
    _fields_ = [("item", DanWorkItem), ("start", _i32), ("n", _i32), ("trunk", _i32), ("past_len", _i32),
                ("past_idx", _i32), ("vt_col", _i32), ("group", _i32), ("reserved", _i32)]


class DanTreeAttnArgs(ctypes.Structure):
    _fields_ = [("abi_version", _i32), ("in_dtype", _i32), ("out_dtype", _i32), ("v_dtype", _i32),
                ("num_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32), ("num_tokens", _i32),
                ("scale", _f32),
                ("q", _vp), ("q_stride_tok", _i64), ("q_stride_head", _i64),
                ("k", _vp), ("k_stride_tok", _i64), ("k_stride_head", _i64),
                ("v", _vp), ("v_stride_tok", _i64), ("v_stride_head", _i64),
                ("out", _vp), ("o_stride_tok", _i64), ("o_stride_head", _i64),
                ("q_scale", _vp), ("k_scale", _vp), ("v_scale", _vp),
                ("segments", _vp), ("num_segments", _i32),
                ("pasts", _vp), ("num_pasts", _i32),
                ("work", _vp), ("num_work", _i32),
                ("key_lo", _vp),
                ("tile_q", _i32), ("vt_cols", _i32),
                ("col_seg", _vp),
                ("workspace", _vp), ("workspace_bytes", _i64), ("phases", _i32),
                ("units", _vp), ("sched_off", _vp), ("num_slots", _i32), ("counts", _vp)]


STAGE_PARTIALS = 1024  # DAN_TREE_ATTN_STAGE_PARTIALS


class DanStageF16Args(ctypes.Structure):
    _fields_ = [("abi_version", _i32), ("d0", _i32), ("d1", _i32), ("d2", _i32), ("x", _vp),
                ("stride0", _i64), ("stride1", _i64), ("out", _vp), ("scale", _vp), ("partial", _vp)]


FRONT_ABI_VERSION = 1
FRONT_NORM_NONE, FRONT_NORM_RMS, FRONT_NORM_RMS_ZERO_CENTERED = 0, 1, 2


class DanFrontSave(ctypes.Structure):
    _fields_ = [("start", _i32), ("len", _i32), ("k_dst", _vp), ("v_dst", _vp)]


class DanQkvFrontArgs(ctypes.Structure):
    _fields_ = [("abi_version", _i32), ("dtype", _i32), ("num_tokens", _i32), ("num_heads", _i32),
                ("num_kv_heads", _i32), ("head_dim", _i32), ("rotary_dim", _i32), ("norm", _i32), ("eps", _f32),
                ("q", _vp), ("q_stride_tok", _i64), ("q_stride_head", _i64),
                ("k", _vp), ("k_stride_tok", _i64), ("k_stride_head", _i64),
                ("v", _vp), ("v_stride_tok", _i64), ("v_stride_head", _i64),
                ("cos", _vp), ("sin", _vp), ("cs_stride_tok", _i64),
                ("q_norm_weight", _vp), ("k_norm_weight", _vp),
                ("q_out", _vp), ("qo_stride_tok", _i64), ("qo_stride_head", _i64),
                ("k_out", _vp), ("ko_stride_tok", _i64), ("ko_stride_head", _i64),
                ("save_of", _vp), ("saves", _vp), ("num_saves", _i32)]


PLAN_ABI_VERSION = 2
PLAN_MAX_WORK, PLAN_MAX_SLOTS, PLAN_MAX_SEGMENTS, PLAN_MAX_BRANCHES = 4096, 256, 1024, 4096


class DanTreePlanArgs(ctypes.Structure):
    _fields_ = [("abi_version", _i32), ("num_tokens", _i32), ("num_segments", _i32), ("num_branches", _i32),
                ("num_work", _i32), ("num_cols", _i32), ("tile_q", _i32), ("groups", _i32), ("num_cus", _i32),
                ("overhead", _i32),
                ("segments", _vp), ("branch_starts", _vp),
                ("key_lo", _vp), ("col_seg", _vp), ("work", _vp), ("cost", _vp), ("units", _vp), ("sched_off", _vp),
                ("counts", _vp)]


FP8_ABI_VERSION = 2
FP8_SCALE_TENSOR, FP8_SCALE_ROW = 0, 1
FP8_GEMM_X_SCALE_TENSOR, FP8_GEMM_W_SCALE_TENSOR, FP8_GEMM_X_TILED, FP8_GEMM_W_TILED = 1, 2, 4, 8
FP8_LAYOUT_ROWS, FP8_LAYOUT_TILED = 0, 1


class DanFp8QuantArgs(ctypes.Structure):
    _fields_ = [("abi_version", _i32), ("dtype", _i32), ("rows", _i32), ("cols", _i32), ("mode", _i32),
                ("layout", _i32), ("x", _vp), ("x_stride", _i64), ("xq", _vp), ("scale", _vp)]


class DanFp8GemmArgs(ctypes.Structure):
    _fields_ = [("abi_version", _i32), ("out_dtype", _i32), ("m", _i32), ("n", _i32), ("k", _i32), ("flags", _i32),
                ("xq", _vp), ("xq_stride", _i64), ("x_scale", _vp), ("wq", _vp), ("wq_stride", _i64),
                ("w_scale", _vp), ("bias", _vp), ("y", _vp), ("y_stride", _i64)]


GDN_ABI_VERSION = 4
GDN_FORM_TOKEN, GDN_FORM_CHUNK = 0, 1
GDN_CHUNK = 64


class DanGdnArgs(ctypes.Structure):
    _fields_ = [("abi_version", _i32), ("dtype", _i32), ("num_k_heads", _i32), ("num_v_heads", _i32), ("k_dim", _i32),
                ("v_dim", _i32), ("num_runs", _i32), ("num_tokens", _i32), ("cu", _vp),
                ("q", _vp), ("q_stride_tok", _i64), ("q_stride_head", _i64),
                ("k", _vp), ("k_stride_tok", _i64), ("k_stride_head", _i64),
                ("v", _vp), ("v_stride_tok", _i64), ("v_stride_head", _i64),
                ("g", _vp), ("beta", _vp), ("states_in", _vp), ("states_out", _vp),
                ("out", _vp), ("o_stride_tok", _i64), ("o_stride_head", _i64),
                ("workspace", _vp), ("workspace_bytes", _i64), ("form", _i32), ("reserved", _i32),
                ("state_index", _vp), ("num_states_in", _i32), ("reserved2", _i32)]


class DanGdnConvArgs(ctypes.Structure):
    _fields_ = [("abi_version", _i32), ("dtype", _i32), ("channels", _i32), ("kernel", _i32), ("num_rows", _i32),
                ("num_hist_rows", _i32), ("num_ext", _i32), ("num_out", _i32),
                ("src", _vp), ("src_stride", _i64), ("hist", _vp), ("ext", _vp), ("take", _vp), ("weight", _vp),
                ("out", _vp), ("out_stride", _i64), ("num_heads", _i32), ("reserved", _i32), ("rows", _vp),
                ("b", _vp), ("b_stride", _i64), ("a", _vp), ("a_stride", _i64), ("a_log", _vp), ("dt_bias", _vp),
                ("beta", _vp), ("g", _vp)]


EXPORTS = ("dan_tree_attn_fwd", "dan_tree_attn_fwd_noalloc", "dan_tree_attn_stage_f16", "dan_tree_attn_tile_q", "dan_tree_attn_head_groups", "dan_tree_attn_workspace_size",
           "dan_tree_attn_last_error", "dan_tree_attn_abi_version", "dan_qkv_front", "dan_qkv_front_abi_version",
           "dan_tree_attn_plan", "dan_tree_attn_plan_slots", "dan_tree_attn_plan_abi_version",
           "dan_fp8_quantize", "dan_fp8_gemm", "dan_fp8_tiled_bytes", "dan_fp8_abi_version", "dan_gdn_fwd", "dan_gdn_workspace_size", "dan_gdn_abi_version",
           "dan_gdn_conv")

_lock = threading.Lock()
_lib = None


def load(path=LIB_PATH):
    """Load the library (once) and declare its signatures. Raises RuntimeError
    when it is missing, unloadable or speaks another ABI version."""
    global _lib
    with _lock:
        if _lib is not None and path == LIB_PATH:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built; run __graft_entry__.build() (hipcc for gfx950)")
        import torch  # noqa: F401  -- torch's HIP runtime must be loaded first (shared soname)

        lib = ctypes.CDLL(path, mode=ctypes.RTLD_LOCAL)
        lib.dan_tree_attn_fwd.argtypes = [ctypes.POINTER(DanTreeAttnArgs), _vp]
        lib.dan_tree_attn_fwd.restype = ctypes.c_int
        lib.dan_tree_attn_fwd_noalloc.argtypes = [ctypes.POINTER(DanTreeAttnArgs), _vp]
        lib.dan_tree_attn_fwd_noalloc.restype = ctypes.c_int
        lib.dan_tree_attn_stage_f16.argtypes = [ctypes.POINTER(DanStageF16Args), _vp]
        lib.dan_tree_attn_stage_f16.restype = ctypes.c_int
        lib.dan_tree_attn_tile_q.argtypes = [_i32, _i32, _i32]
        lib.dan_tree_attn_tile_q.restype = ctypes.c_int
        lib.dan_tree_attn_head_groups.argtypes = [_i32, _i32]
        lib.dan_tree_attn_head_groups.restype = ctypes.c_int
        lib.dan_tree_attn_workspace_size.argtypes = [_i32, _i32, _i32]
        lib.dan_tree_attn_workspace_size.restype = _i64
        lib.dan_tree_attn_last_error.argtypes = []
        lib.dan_tree_attn_last_error.restype = ctypes.c_char_p
        lib.dan_tree_attn_abi_version.argtypes = []
        lib.dan_tree_attn_abi_version.restype = ctypes.c_int
        lib.dan_qkv_front.argtypes = [ctypes.POINTER(DanQkvFrontArgs), _vp]
        lib.dan_qkv_front.restype = ctypes.c_int
        lib.dan_qkv_front_abi_version.argtypes = []
        lib.dan_qkv_front_abi_version.restype = ctypes.c_int
        lib.dan_tree_attn_plan.argtypes = [ctypes.POINTER(DanTreePlanArgs), _vp]
        lib.dan_tree_attn_plan.restype = ctypes.c_int
        lib.dan_tree_attn_plan_slots.argtypes = [_i32, _i32, _i32]
        lib.dan_tree_attn_plan_slots.restype = ctypes.c_int
        lib.dan_tree_attn_plan_abi_version.argtypes = []
        lib.dan_tree_attn_plan_abi_version.restype = ctypes.c_int
        lib.dan_fp8_quantize.argtypes = [ctypes.POINTER(DanFp8QuantArgs), _vp]
        lib.dan_fp8_quantize.restype = ctypes.c_int
        lib.dan_fp8_gemm.argtypes = [ctypes.POINTER(DanFp8GemmArgs), _vp]
        lib.dan_fp8_gemm.restype = ctypes.c_int
        lib.dan_fp8_tiled_bytes.argtypes = [_i32, _i32]
        lib.dan_fp8_tiled_bytes.restype = _i64
        lib.dan_fp8_abi_version.argtypes = []
        lib.dan_fp8_abi_version.restype = ctypes.c_int
        lib.dan_gdn_fwd.argtypes = [ctypes.POINTER(DanGdnArgs), _vp]
        lib.dan_gdn_fwd.restype = ctypes.c_int
        lib.dan_gdn_workspace_size.argtypes = [_i32, _i32, _i32, _i32, _i32, _i32]
        lib.dan_gdn_workspace_size.restype = _i64
        lib.dan_gdn_conv.argtypes = [ctypes.POINTER(DanGdnConvArgs), _vp]
        lib.dan_gdn_conv.restype = ctypes.c_int
        lib.dan_gdn_abi_version.argtypes = []
        lib.dan_gdn_abi_version.restype = ctypes.c_int
        got = (lib.dan_tree_attn_abi_version(), lib.dan_qkv_front_abi_version(), lib.dan_tree_attn_plan_abi_version(),
               lib.dan_fp8_abi_version(), lib.dan_gdn_abi_version())
        want = (ABI_VERSION, FRONT_ABI_VERSION, PLAN_ABI_VERSION, FP8_ABI_VERSION, GDN_ABI_VERSION)
        if got != want:
            raise RuntimeError(f"{path} speaks ABI versions {got} (attention, front end, planner, fp8, delta rule), this package "
                               f"{want}; rebuild it")
        if path == LIB_PATH:
            _lib = lib
        return lib


def last_error(lib):
    msg = lib.dan_tree_attn_last_error()
    return msg.decode() if msg else ""


def tile_q(num_heads, num_kv_heads, head_dim=128, *, lib=None):
    """Queries per work item the kernel expects (0: unsupported head layout)."""
    return (lib or load()).dan_tree_attn_tile_q(num_heads, num_kv_heads, head_dim)


def head_groups(num_heads, num_kv_heads, lib=None):
    """Head groups of the persistent schedule (0: unsupported head layout)."""
    return (lib or load()).dan_tree_attn_head_groups(num_heads, num_kv_heads)


def workspace_size(num_kv_heads, head_dim, vt_cols, lib=None):
    """Bytes of device workspace one launch needs (0: invalid arguments)."""
    return (lib or load()).dan_tree_attn_workspace_size(num_kv_heads, head_dim, vt_cols)


def stage_f16(args, stream, lib=None):
    """Launch the fp32 -> fp16 staging; raises RuntimeError on failure."""
    lib = lib or load()
    rc = lib.dan_tree_attn_stage_f16(ctypes.byref(args), _vp(stream))
    if rc != OK:
        raise RuntimeError(f"dan_tree_attn_stage_f16 failed (status {rc}): {last_error(lib)}")


def forward(args, stream, lib=None):
    """Launch; raises RuntimeError with the library's message on failure."""
    lib = lib or load()
    rc = lib.dan_tree_attn_fwd(ctypes.byref(args), _vp(stream))
    if rc != OK:
        raise RuntimeError(f"dan_tree_attn_fwd failed (status {rc}): {last_error(lib)}")


def forward_noalloc(args, stream, lib=None):
    """Launch through dan_tree_attn_fwd_noalloc (the V^T copy in the library's
    own scratch, nothing allocated); raises RuntimeError on failure."""
    lib = lib or load()
    rc = lib.dan_tree_attn_fwd_noalloc(ctypes.byref(args), _vp(stream))
    if rc != OK:
        raise RuntimeError(f"dan_tree_attn_fwd_noalloc failed (status {rc}): {last_error(lib)}")


def front(args, stream, lib=None):
    """Launch the attention front end; raises RuntimeError with the library's message on failure."""
    lib = lib or load()
    rc = lib.dan_qkv_front(ctypes.byref(args), _vp(stream))
    if rc != OK:
        raise RuntimeError(f"dan_qkv_front failed ({rc}): {last_error(lib)}")


def plan_slots(num_work, groups, num_cus, lib=None):
    """Slots of the device planner's schedule (0: invalid arguments)."""
    return (lib or load()).dan_tree_attn_plan_slots(num_work, groups, num_cus)


def plan(args, stream, lib=None):
    """Launch the device-side tile planner; raises RuntimeError with the library's message on failure."""
    lib = lib or load()
    rc = lib.dan_tree_attn_plan(ctypes.byref(args), _vp(stream))
    if rc != OK:
        raise RuntimeError(f"dan_tree_attn_plan failed ({rc}): {last_error(lib)}")


def fp8_quantize(args, stream, lib=None):
    """Launch the e4m3 quantizer; raises RuntimeError with the library's message on failure."""
    lib = lib or load()
    rc = lib.dan_fp8_quantize(ctypes.byref(args), _vp(stream))
    if rc != OK:
        raise RuntimeError(f"dan_fp8_quantize failed ({rc}): {last_error(lib)}")


def fp8_tiled_bytes(rows, cols, lib=None):
    """Bytes of an [rows, cols] e4m3 tensor in the GEMM's tiled layout."""
    return (lib or load()).dan_fp8_tiled_bytes(rows, cols)


def fp8_gemm(args, stream, lib=None):
    """Launch the e4m3 GEMM; raises RuntimeError with the library's message on failure."""
    lib = lib or load()
    rc = lib.dan_fp8_gemm(ctypes.byref(args), _vp(stream))
    if rc != OK:
        raise RuntimeError(f"dan_fp8_gemm failed ({rc}): {last_error(lib)}")


def gdn(args, stream, lib=None):
    """Launch the gated delta rule; raises RuntimeError with the library's message on failure."""
    lib = lib or load()
    rc = lib.dan_gdn_fwd(ctypes.byref(args), _vp(stream))
    if rc != OK:
        raise RuntimeError(f"dan_gdn_fwd failed ({rc}): {last_error(lib)}")


def gdn_conv(args, stream, lib=None):
    """Launch the conv and gates of one DeltaNet phase; raises RuntimeError with the library's message on failure."""
    lib = lib or load()
    rc = lib.dan_gdn_conv(ctypes.byref(args), _vp(stream))
    if rc != OK:
        raise RuntimeError(f"dan_gdn_conv failed ({rc}): {last_error(lib)}")
