"""Random-init ViT backbone weights and inputs at any size, shared by the
oracle, GPU and golden tests: Xavier-uniform linear weights, PyTorch's
default U(+-1/sqrt(fan_in)) biases, LayerNorm affine near (1, 0)."""
import math

import numpy as np


def xavier(g, out_f, in_f):
    b = math.sqrt(6.0 / (in_f + out_f))
    return g.uniform(-b, b, (out_f, in_f)).astype(np.float32)


def bias(g, n, fan_in):
    b = 1.0 / math.sqrt(fan_in)
    return g.uniform(-b, b, n).astype(np.float32)


def block_weights(g, E, mlp, window):
    return {
        "n1w": (1 + 0.1 * g.standard_normal(E)).astype(np.float32),
        "n1b": (0.1 * g.standard_normal(E)).astype(np.float32),
        "qkvw": xavier(g, 3 * E, E), "qkvb": bias(g, 3 * E, E),
        "projw": xavier(g, E, E), "projb": bias(g, E, E),
        "n2w": (1 + 0.1 * g.standard_normal(E)).astype(np.float32),
        "n2b": (0.1 * g.standard_normal(E)).astype(np.float32),
        "l1w": xavier(g, mlp, E), "l1b": bias(g, mlp, E),
        "l2w": xavier(g, E, mlp), "l2b": bias(g, E, mlp),
        "window": window,
    }


def trunk_case(seed, grid, ps, E, mlp, windows, pt=None):
    """Image (ImageNet-style (u - 0.5) / 0.5 of U(0, 1)), patch weight
    [E, 3 ps^2], position embedding of a pt x pt pretraining grid tiled
    over the grid [grid^2, E] (pt 2, or 1 for an odd grid, unless given),
    ln_pre and one weight dict per entry of `windows` (window side, 0 =
    global)."""
    g = np.random.default_rng(seed)
    side = grid * ps
    img = ((g.random((3, side, side), dtype=np.float32) - 0.5) / 0.5)
    pe_w = xavier(g, E, 3 * ps * ps)
    if pt is None:
        pt = 2 if grid % 2 == 0 else 1
    pe = (0.02 * g.standard_normal((pt * pt, E))).astype(np.float32)
    yy, xx = np.divmod(np.arange(grid * grid), grid)
    pos = pe[(yy % pt) * pt + xx % pt]
    lnpw = (1 + 0.1 * g.standard_normal(E)).astype(np.float32)
    lnpb = (0.1 * g.standard_normal(E)).astype(np.float32)
    blocks = [block_weights(g, E, mlp, w) for w in windows]
    return img, pe_w, np.ascontiguousarray(pos), lnpw, lnpb, blocks
