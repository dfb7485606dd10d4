"""Writes the golden vectors of the attention path from the reference's own
kernels: sam3_kernels.cl compiled unchanged for gfx950 (oracle/ref.mk) and
launched through the ROCm OpenCL runtime the way sam3_model.c launches
them (oracle/ref_harness.c). Run on a machine with an OpenCL GPU device:

    python tests/golden/gen_golden.py OUTDIR [CASE ...]

Each case is one .npz: the reference outputs (full, or sampled rows for
large cases, with the sample indices), plus the SHA-1 of the inputs. The
inputs are not stored: golden_cases.py regenerates them from fixed seeds
(numpy PCG64, platform independent) and the tests check the SHA-1.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, HERE)

from oracle import refk  # noqa: E402
import golden_cases as gc  # noqa: E402


def sha(*arrays):
    h = hashlib.sha1()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main(out, names=None):
    os.makedirs(out, exist_ok=True)
    print("reference device:", refk.device(), flush=True)
    for name, make in gc.CASES.items():
        if names and name not in names:
            continue
        case = make()
        res = gc.run_reference(name, case, refk)
        rows = case.get("sample_rows")
        payload = {k: (v[rows] if rows is not None and v.ndim == 2 else v)
                   for k, v in res.items()}
        if rows is not None:
            payload["sample_rows"] = rows
        np.savez_compressed(os.path.join(out, name + ".npz"),
                            input_sha1=np.array(sha(*case["inputs"])),
                            **payload)
        print("wrote", name, {k: v.shape for k, v in payload.items()},
              flush=True)


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2:])
