"""Shared helpers of the GPU parity tests: seeded inputs of the named
workloads and oracle computations restricted to sampled rows."""
import math

import numpy as np

from oracle import oracle as orc


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def max_abs(got, want):
    return float(np.abs(np.asarray(got, np.float64) -
                        np.asarray(want, np.float64)).max())


def report(name, got, want):
    r, a = rel_l2(got, want), max_abs(got, want)
    print("%s: rel-L2 %.3e max-abs %.3e" % (name, r, a), flush=True)
    return r


def block_inputs(seed, grid=72, E=1024):
    """x ~ N(0,1) [grid^2, E]; LayerNorm gamma 1, beta 0; Xavier-uniform
    QKV weight [3E, E]; bias ~ U(+-1/sqrt(E)) (PyTorch's Linear default)."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((grid * grid, E), dtype=np.float32)
    n1w = np.ones(E, np.float32)
    n1b = np.zeros(E, np.float32)
    bound = math.sqrt(6.0 / (E + 3 * E))
    w = g.uniform(-bound, bound, (3 * E, E)).astype(np.float32)
    b = g.uniform(-1 / math.sqrt(E), 1 / math.sqrt(E), 3 * E).astype(np.float32)
    return x, n1w, n1b, w, b


def oracle_attn_rows(qkv_unit, E, head, rows, table=None, scale=0.125):
    """Attention output [len(rows), 64] of `rows` of one unit (N rows of
    the fused qkv layout), by the reference's profile=cpu sequence:
    rope_apply, gemm_cpu_t (Q K^T, alpha scale), softmax_rows,
    gemm_cpu_n (P V)."""
    N = qkv_unit.shape[0]
    q = qkv_unit if table is None else orc.rope_apply(qkv_unit, E, 64, N, table)
    Q = np.ascontiguousarray(q[rows, head * 64:(head + 1) * 64])
    K = np.ascontiguousarray(q[:, E + head * 64:E + (head + 1) * 64])
    V = np.ascontiguousarray(q[:, 2 * E + head * 64:2 * E + (head + 1) * 64])
    R = len(rows)
    S = np.zeros((R, N), np.float32)
    orc.gemm(orc.GEMM_CPU_T, R, N, 64, Q, 0, 64, 0, 0, K, 0, 64, 0, 0, 1, S, 0,
             N, 0, 0, 1, 1, alpha=scale)
    S = orc.softmax_rows(S)
    O = np.zeros((R, 64), np.float32)
    orc.gemm(orc.GEMM_SEQ, R, 64, N, S, 0, N, 0, 0, V, 0, 64, 0, 0, 0, O, 0, 64,
             0, 0, 1, 1)
    return O
