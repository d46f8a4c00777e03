"""Writes the golden fixtures under tests/golden/ (run from the repo root):

    python tests/golden/make_golden.py

- mask_known_answers.json: the known answers of the reference's only
  known-answer test for this path (tests/test_runner.py:16-22), transcribed
  as data: three rows of tree_mask([0, 0, 1, 1, 2]) and the identity
  branch_rows_mask(b, 3) == tree_mask(b)[3:] for b = [0, 0, 0, 1, 1, 2, 3, 3].
- input_digests.json: SHA-256 of the seeded inputs of every workload, so a
  change of generator (or of numpy's stream) is caught before any parity
  number is trusted.
- bruteforce_samples.npz: fp64 brute-force outputs (the oracle's
  ``attend_bruteforce``) at sampled rows of config 1 and of the reference's
  differential shapes in fp32, to catch drift of the oracle itself.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from dan_amd import workloads as W  # noqa: E402
from oracle import tree_attention as O  # noqa: E402

SAMPLE_ROWS = {"c1": [0, 1, 2, 100, 255, 256, 257, 287, 288, 300, 319, 320, 351, 352, 383],
               "runner_shapes": [0, 39, 40, 44, 45, 53, 54, 55, 61, 62, 91, 92, 97, 98, 161, 162, 174, 175, 191, 192,
                                 206]}


def workloads():
    return {"c1": W.config1(0), "c2": W.config2(0), "c3": W.config3(0), "c4": W.config4(0),
            "runner_shapes": W.runner_shapes(0), "runner_shapes_fp32": W.runner_shapes(0, dtype=torch.float32)}


def main():
    masks = {
        "tree_mask": {"branch": [0, 0, 1, 1, 2],
                      "rows": {"1": [True, True, False, False, False], "3": [True, True, True, True, False],
                               "4": [True, True, False, False, True]}},
        "branch_rows_mask_equals_tree_rows": {"branch": [0, 0, 0, 1, 1, 2, 3, 3], "trunk": 3},
        "source": "tests/test_runner.py:16-22 of the reference",
    }
    with open(os.path.join(HERE, "mask_known_answers.json"), "w") as f:
        json.dump(masks, f, indent=1)

    ws = workloads()
    digests = {name: {"digest": w.digest(), "meta": w.meta} for name, w in ws.items()}
    with open(os.path.join(HERE, "input_digests.json"), "w") as f:
        json.dump(digests, f, indent=1, sort_keys=True)

    samples = {}
    for name, w in (("c1", ws["c1"]), ("runner_shapes", ws["runner_shapes_fp32"])):
        ref = O.attend_bruteforce(w.q, w.k, w.v, w.segments, w.layer)
        rows = SAMPLE_ROWS[name]
        samples[f"{name}_rows"] = np.array(rows)
        samples[f"{name}_out"] = ref[:, rows]
    np.savez_compressed(os.path.join(HERE, "bruteforce_samples.npz"), **samples)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
