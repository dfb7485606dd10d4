"""The CPU oracle against the golden vectors of the reference's own
kernels (tests/golden/vectors, written by tests/golden/gen_golden.py from
sam3_kernels.cl run unchanged through the OpenCL runtime).

Data movement and RoPE must match bit for bit; arithmetic within
rel-L2 1e-6 (the differences are the last bits of the runtimes' exp / erf
and of dot() contraction order, which nothing in the reference pins)."""
import hashlib
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import golden_cases as gc  # noqa: E402

VEC = os.path.join(HERE, "golden", "vectors")
EXACT = {"rope", "window", "convt_plain"}


def load(name):
    case = gc.CASES[name]()
    gold = np.load(os.path.join(VEC, name + ".npz"))
    h = hashlib.sha1()
    for a in case["inputs"]:
        h.update(np.ascontiguousarray(a).tobytes())
    assert h.hexdigest() == str(gold["input_sha1"]), "regenerated inputs differ"
    return case, gold


def compare(name, got, gold, tol):
    rows = gold["sample_rows"] if "sample_rows" in gold.files else None
    for k, v in got.items():
        if rows is not None and v.ndim == 2:
            v = v[rows]
        ref = gold[k]
        if name in EXACT:
            np.testing.assert_array_equal(v, ref)
        else:
            err = np.linalg.norm(v.astype(np.float64) - ref) / np.linalg.norm(ref)
            assert err <= tol, (name, k, err)


@pytest.mark.parametrize("name", [n for n in gc.CASES
                                  if not n.startswith("mask_post")])
def test_oracle_matches_reference_kernels(orc, name):
    case, gold = load(name)
    compare(name, gc.run_reference(name, case, gc.OracleImpl(orc)), gold, 1e-6)


@pytest.mark.parametrize("name", [n for n in gc.CASES if n.startswith("mask_post")])
def test_oracle_mask_post_matches_reference(orc, name):
    """mask_post: the reference divides L / out in OpenCL's default float
    division (2.5 ulp), the oracle (and the HIP kernel) correctly rounded,
    so the interpolated value may differ in its last bits. Masks and counts
    must agree everywhere except at pixels whose exact (float64) value lies
    on a threshold (0, +-offset) within 1e-5; bounding boxes are those of
    the masks."""
    import torch
    case, gold = load(name)
    got = gc.run_reference(name, case, gc.OracleImpl(orc))
    low, sel = case["inputs"]
    off = case["offset"]
    v = torch.nn.functional.interpolate(
        torch.from_numpy(low[sel]).double()[:, None],
        size=(case["out_h"], case["out_w"]), mode="bilinear",
        align_corners=False)[:, 0].numpy()
    diff = got["mask"] != gold["mask"]
    assert np.all(np.abs(v[diff]) < 1e-5)
    for k in range(len(sel)):
        near_i = int((np.abs(v[k] - off) < 1e-5).sum())
        near_u = int((np.abs(v[k] + off) < 1e-5).sum())
        assert abs(int(got["stats"][k, 0]) - int(gold["stats"][k, 0])) <= near_i
        assert abs(int(got["stats"][k, 1]) - int(gold["stats"][k, 1])) <= near_u
        for st, m in ((got["stats"][k], got["mask"][k]),
                      (gold["stats"][k], gold["mask"][k])):
            ys, xs = np.nonzero(m)
            box = [xs.min(), ys.min(), xs.max(), ys.max()] if len(xs) else \
                [0x7fffffff, 0x7fffffff, -1, -1]
            assert list(st[2:]) == box
    if name == "mask_post_random":
        # Away from thresholds the two agree exactly.
        assert diff.sum() == 0


def test_every_case_has_vectors():
    have = {f[:-4] for f in os.listdir(VEC) if f.endswith(".npz")}
    assert have == set(gc.CASES)


@pytest.mark.parametrize("name", [n for n in gc.CASES if n.startswith("attend_")])
def test_oracle_attend_matches_reference(orc, name):
    """or_attend (the composed attend() of the oracle, with its own head
    chunking and GEMM dispatch) against the reference kernels' sequence."""
    case, gold = load(name)
    Q, K, V = case["inputs"][:3]
    kw = {}
    if case["mode"] == "box":
        kw = dict(dy=case["inputs"][3], dx=case["inputs"][4], W=case["W"])
    O = orc.attend(Q, K, V, case["heads"], case["hd"],
                   causal=case["mode"] == "causal", **kw)
    compare(name, {"O": O}, gold, 1e-6)
