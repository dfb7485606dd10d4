"""GPU parity of the fused attention path against the oracle.

Oracle = the reference's profile=cpu operator sequence restated on the
CPU (rope_apply, gemm_cpu_t with alpha 1/8, softmax_rows, gemm_cpu_n).
Bars: rel-L2 <= 2e-5 for the fp32 path, <= 2e-2 for the bf16 path; the
max-abs error is printed with every check.

Full-size workloads (9 x 576 windows, 5184 global tokens) are checked on
sampled (unit, head, query-row) sets: on the fp32 path the QKV projection
rows against the oracle's LayerNorm + linear and the attention rows
against the oracle's attention computed from the device's qkv; on the
bf16 path (whose projection packs the attention operands in its store and
writes no fp32 qkv) the attention rows against the oracle's attention of
the oracle's qkv.
"""
import math

import numpy as np
import pytest

from gpu_common import block_inputs, oracle_attn_rows, rel_l2, report

pytestmark = pytest.mark.gpu

TOL = {"fp32": 2e-5, "bf16": 2e-2}


@pytest.fixture(scope="module")
def hip():
    import sam3_hip
    return sam3_hip


@pytest.fixture(scope="module", params=["fp32", "bf16"])
def be(hip, request):
    b = hip.Backend(precision=request.param)
    b.precision = request.param
    yield b
    b.free()


def _oracle_units(orc, qkv, N, nunits, heads, E, table):
    """Oracle attention of every (unit, head) of a [nunits * N, 3E] qkv."""
    out = np.zeros((nunits * N, E), np.float32)
    for u in range(nunits):
        unit = qkv[u * N:(u + 1) * N]
        for h in range(heads):
            out[u * N:(u + 1) * N, h * 64:(h + 1) * 64] = oracle_attn_rows(
                unit, E, h, np.arange(N), table)
    return out


def test_single_window(hip, be, orc):
    """One 576-token window, 16 heads x 64, N(0,1), no mask, no RoPE."""
    N, H, E = 576, 16, 1024
    m = hip.Model(be, embed=E, heads=H)
    qkv = np.random.default_rng(11).standard_normal((N, 3 * E), np.float32)
    dq = be.upload(qkv)
    do = be.alloc(N * E * 4)
    hip.attn_fused(m, N, H, H, hip.bmat(dq, 0, 3 * E, 0, 64),
                   hip.bmat(dq, E, 3 * E, 0, 64),
                   hip.bmat(dq, 2 * E, 3 * E, 0, 64),
                   hip.bmat(do, 0, E, 0, 64), None, 1, 0.125)
    got = be.read(do).reshape(N, E)
    want = _oracle_units(orc, qkv, N, 1, H, E, None)
    assert report("single window %s" % be.precision, got, want) <= TOL[be.precision]
    be.release(dq)
    be.release(do)


def test_split_launch_repeats(hip, be, orc):
    """Launch-starved shapes merge their key splits inside the one launch
    (the exact path: 3 splits of the window's tiles, folded in order by the
    last to arrive; 10 splits of the 1000-token tiles, in groups of 8 and
    2 and then across the groups; bf16: key groups inside the workgroup).
    The same bits on every launch, and each launch leaves its arrival
    counts at zero for the next one of another tile count: one 576-token
    window of 16 heads, then 1000 tokens of 2 heads with RoPE, then the
    window again."""
    N, H, E = 576, 16, 1024
    m = hip.Model(be, embed=E, heads=H)
    qkv = np.random.default_rng(12).standard_normal((N, 3 * E), np.float32)
    dq = be.upload(qkv)
    do = be.alloc(N * E * 4)

    def window():
        hip.attn_fused(m, N, H, H, hip.bmat(dq, 0, 3 * E, 0, 64),
                       hip.bmat(dq, E, 3 * E, 0, 64),
                       hip.bmat(dq, 2 * E, 3 * E, 0, 64),
                       hip.bmat(do, 0, E, 0, 64), None, 1, 0.125)
        return be.read(do).reshape(N, E)

    first = window()
    want = _oracle_units(orc, qkv, N, 1, H, E, None)
    assert report("split window %s" % be.precision, first, want) <= TOL[be.precision]

    N2, H2, E2 = 1000, 2, 128
    table = orc.rope_table(32)[:N2]
    qkv2 = np.random.default_rng(13).standard_normal((N2, 3 * E2), np.float32)
    dq2, dt = be.upload(qkv2), be.upload(table)
    do2 = be.alloc(N2 * E2 * 4)
    hip.attn_fused(m, N2, H2, H2, hip.bmat(dq2, 0, 3 * E2, 0, 64),
                   hip.bmat(dq2, E2, 3 * E2, 0, 64),
                   hip.bmat(dq2, 2 * E2, 3 * E2, 0, 64),
                   hip.bmat(do2, 0, E2, 0, 64), dt, N2, 0.125)
    got2 = be.read(do2).reshape(N2, E2)
    want2 = _oracle_units(orc, qkv2, N2, 1, H2, E2, table)
    assert report("split 1000 x 2 %s" % be.precision, got2, want2) <= TOL[be.precision]

    for _ in range(3):
        assert np.array_equal(window(), first)
    for x in (dq, do, dq2, dt, do2):
        be.release(x)
    m.free()


@pytest.mark.parametrize("N,nunits", [(37, 3), (100, 2), (200, 1), (64, 2)])
def test_rope_and_ragged_lengths(hip, be, orc, N, nunits):
    """Token counts that are not multiples of the 32/64-key blocks or the
    128-query tiles, RoPE on Q and K, several units with batch strides."""
    H, E = 2, 128
    m = hip.Model(be, embed=E, heads=H)
    side = math.isqrt(N)
    table = orc.rope_table(side + 1)[:N] if side * side != N else orc.rope_table(side)
    qkv = np.random.default_rng(N).standard_normal((nunits * N, 3 * E), np.float32)
    dq, dt = be.upload(qkv), be.upload(table)
    do = be.alloc(nunits * N * E * 4)
    st = N * 3 * E
    hip.attn_fused(m, N, nunits * H, H, hip.bmat(dq, 0, 3 * E, st, 64),
                   hip.bmat(dq, E, 3 * E, st, 64),
                   hip.bmat(dq, 2 * E, 3 * E, st, 64),
                   hip.bmat(do, 0, E, N * E, 64), dt, N, 0.125)
    got = be.read(do).reshape(nunits * N, E)
    want = _oracle_units(orc, qkv, N, nunits, H, E, table)
    assert report("ragged N=%d %s" % (N, be.precision), got, want) <= TOL[be.precision]


@pytest.mark.parametrize("N,nunits,H", [(576, 1, 16), (700, 1, 2), (300, 3, 1)])
def test_grouped_launch(hip, be, orc, N, nunits, H):
    """Shapes whose query tiles leave the device launch-starved take, on
    the bf16 path, one launch whose workgroups split the key blocks
    between groups of waves and merge them in LDS in group order (no
    records in memory): one 576-token window of 16 heads (four
    groups of 64-query tiles, every key block resident in LDS), 700 tokens
    (four double-buffered groups; 60 keys in the last block, 60 queries in
    the last tile) and 300 tokens (two groups of 128-query tiles; 44 keys
    in the last block). The exact path splits the 32-key blocks across
    workgroups and merges their records inside the launch. Every row
    against the oracle, and a relaunch gives the same bits."""
    E = 64 * H
    m = hip.Model(be, embed=E, heads=H)
    side = math.isqrt(N)
    table = orc.rope_table(side) if side * side == N else orc.rope_table(side + 1)[:N]
    qkv = np.random.default_rng(N + H).standard_normal((nunits * N, 3 * E), np.float32)
    dq, dt = be.upload(qkv), be.upload(table)
    do = be.alloc(nunits * N * E * 4)
    st = N * 3 * E
    print("grouped N=%d units=%d %s" % (N, nunits * H, be.precision), flush=True)

    def launch():
        hip.attn_fused(m, N, nunits * H, H, hip.bmat(dq, 0, 3 * E, st, 64),
                       hip.bmat(dq, E, 3 * E, st, 64),
                       hip.bmat(dq, 2 * E, 3 * E, st, 64),
                       hip.bmat(do, 0, E, N * E, 64), dt, N, 0.125)
        return be.read(do).reshape(nunits * N, E)

    got = launch()
    if be.precision == "bf16":
        # No key-split partials were allocated: the grouped launch ran.
        assert not m.m.apart
    want = _oracle_units(orc, qkv, N, nunits, H, E, table)
    assert report("grouped N=%d %s" % (N, be.precision), got, want) <= TOL[be.precision]
    assert np.array_equal(launch(), got)
    be.release(dq)
    be.release(dt)
    be.release(do)


@pytest.mark.parametrize("N,imgs,H,balanced", [
    (1024, 5, 16, True), (961, 5, 13, False), (1795, 1, 37, True),
    (1027, 2, 29, True)])
def test_many_units(hip, be, orc, N, imgs, H, balanced):
    """imgs images x H heads of N tokens (RoPE), every row against the
    oracle, and a second launch bit-identical to the first. On a 256-CU
    device (8 XCDs of 32 CUs) the bf16 path takes its balanced launch when
    an XCD's share of the 128-query tiles lies strictly between two and
    three per CU: two whole tiles per CU, the rest's key blocks shared by
    one more workgroup per CU, the pieces of a tile cut between them
    merged by the last to arrive, in piece order.
    - 1024 tokens, 80 units: 640 tiles, 80 per XCD, 16 full key blocks.
    - 961 tokens, 65 units: 520 ragged tiles (65 queries in the last, one
      key in the last block); one tile over the whole ones per XCD has
      16 pairs for 32 sharing workgroups, so the plain grid runs.
    - 1795 tokens, 37 units: 555 tiles (not a multiple of 8), 70 per XCD
      and 65 on the last, whose one shared tile's 29 key blocks are fewer
      than 32 sharing workgroups (one per pair there); 3 keys in the last
      key block, 3 queries in the last tile.
    - 1027 tokens, 58 units: 522 tiles, 66 per XCD, 60 on the last (fewer
      than its 64 whole-tile workgroups: nothing shared there); 3 keys in
      the last block."""
    E = 64 * H
    m = hip.Model(be, embed=E, heads=H)
    side = math.isqrt(N)
    table = orc.rope_table(side) if side * side == N else orc.rope_table(side + 1)[:N]
    qkv = np.random.default_rng(77).standard_normal((imgs * N, 3 * E), np.float32)
    dq, dt = be.upload(qkv), be.upload(table)
    do = be.alloc(imgs * N * E * 4)
    st = N * 3 * E
    print("many units N=%d units=%d %s" % (N, imgs * H, be.precision), flush=True)

    def launch():
        hip.attn_fused(m, N, imgs * H, H, hip.bmat(dq, 0, 3 * E, st, 64),
                       hip.bmat(dq, E, 3 * E, st, 64),
                       hip.bmat(dq, 2 * E, 3 * E, st, 64),
                       hip.bmat(do, 0, E, N * E, 64), dt, N, 0.125)
        return be.read(do).reshape(imgs * N, E)

    got = launch()
    if be.precision == "bf16" and be.cu_count == 256:
        # The balanced launch allocates its piece records on first use.
        assert bool(m.m.askrec) == balanced
    want = _oracle_units(orc, qkv, N, imgs, H, E, table)
    assert report("many units %s" % be.precision, got, want) <= TOL[be.precision]
    # A second launch reuses the cut tiles' counters and records (the last
    # piece to arrive resets its tile's counter); the merge's order does
    # not depend on which piece arrives last, so the bits repeat.
    again = launch()
    assert np.array_equal(again, got)
    be.release(dq)
    be.release(dt)
    be.release(do)


@pytest.mark.parametrize("ooff,ldo", [(1, 131), (4, 132), (8, 136)])
def test_output_offsets(hip, be, orc, ooff, ldo):
    """Output rows at an offset and stride that break 16-byte alignment
    (per-element stores) or keep it (rows transposed through LDS), with
    the padding columns between rows left untouched."""
    N, H, E = 150, 2, 128
    m = hip.Model(be, embed=E, heads=H)
    qkv = np.random.default_rng(ooff).standard_normal((N, 3 * E), np.float32)
    dq = be.upload(qkv)
    fill = np.full(ooff + N * ldo, 7.0, np.float32)
    do = be.upload(fill)
    hip.attn_fused(m, N, H, H, hip.bmat(dq, 0, 3 * E, 0, 64),
                   hip.bmat(dq, E, 3 * E, 0, 64),
                   hip.bmat(dq, 2 * E, 3 * E, 0, 64),
                   hip.bmat(do, ooff, ldo, 0, 64), None, 1, 0.125)
    raw = be.read(do)
    got = raw[ooff:].reshape(N, ldo)
    want = _oracle_units(orc, qkv, N, 1, H, E, None)
    assert np.all(raw[:ooff] == 7.0) and np.all(got[:, E:] == 7.0)
    assert report("offsets %d/%d %s" % (ooff, ldo, be.precision), got[:, :E],
                  want) <= TOL[be.precision]
    be.release(dq)
    be.release(do)


def test_attention_closed_forms(hip, be):
    """Zero queries give the mean of V; one token gives V itself."""
    E, H = 128, 2
    m = hip.Model(be, embed=E, heads=H)
    for N in (1, 300):
        qkv = np.random.default_rng(N).standard_normal((N, 3 * E), np.float32)
        qkv[:, :E] = 0.0
        dq = be.upload(qkv)
        do = be.alloc(N * E * 4)
        hip.attn_fused(m, N, H, H, hip.bmat(dq, 0, 3 * E, 0, 64),
                       hip.bmat(dq, E, 3 * E, 0, 64),
                       hip.bmat(dq, 2 * E, 3 * E, 0, 64),
                       hip.bmat(do, 0, E, 0, 64), None, 1, 0.125)
        got = be.read(do).reshape(N, E)
        want = np.broadcast_to(qkv[:, 2 * E:].astype(np.float64).mean(0), (N, E))
        tol = 1e-6 if be.precision == "fp32" else 1e-2
        assert rel_l2(got, want) <= tol


def _vit_small(hip, be, orc, grid, ws, unfused=False, E=128):
    H = E // 64
    x, n1w, n1b, w, b = block_inputs(grid + ws, grid, E)
    s = ws if ws else grid
    table = orc.rope_table(s)
    blk = hip.VitBlock()
    blk.n1w, blk.n1b = be.upload(n1w), be.upload(n1b)
    blk.qkvw, blk.qkvb = be.upload_weight(w), be.upload(b)
    blk.window = ws
    m = hip.Model(be, grid=grid, embed=E, heads=H, blocks=[blk])
    if ws:
        m.m.rope_win = be.upload(table)
    else:
        m.m.rope_glob = be.upload(table)
    be.write(m.m.x, 0, x)
    hip.vit_attention(m, blk, unfused)
    nwx = -(-grid // s)
    rows = nwx * nwx * s * s
    got = be.read(m.m.attn, rows * E).reshape(rows, E)
    want = orc.vit_attention(x, grid, E, H, 64, ws, n1w, n1b, w, b, table)
    m.free()
    return got, want


@pytest.mark.parametrize("grid,ws", [(12, 6), (12, 0), (10, 4), (16, 8), (16, 0),
                                     (8, 0), (24, 8)])
@pytest.mark.parametrize("unfused", [False, True])
def test_vit_attention_small(hip, be, orc, grid, ws, unfused):
    """Token counts per unit of 36, 144, 16 (packing kernel on the bf16
    path) and 64, 256, 576 (operands packed by the projection's store;
    grid 8 and 24 leave a partial 128-row tile)."""
    got, want = _vit_small(hip, be, orc, grid, ws, unfused)
    assert report("vit_attention grid=%d ws=%d unfused=%d %s" %
                  (grid, ws, unfused, be.precision), got, want) <= TOL[be.precision]


_FULL_REGION = {}


def _full_region_oracle(orc, ws):
    """Inputs of the full-size region (72 x 72 grid, width 1024, 16 heads)
    and the oracle's whole output for them, computed once per ws."""
    if ws not in _FULL_REGION:
        grid, E, H = 72, 1024, 16
        x, n1w, n1b, w, b = block_inputs(7 + ws, grid, E)
        s = ws if ws else grid
        table = orc.rope_table(s)
        want = orc.vit_attention(x, grid, E, H, 64, ws, n1w, n1b, w, b, table,
                                 cpu=True)
        _FULL_REGION[ws] = (x, n1w, n1b, w, b, table, want)
    return _FULL_REGION[ws]


@pytest.mark.parametrize("ws", [24, 0])
def test_vit_attention_full_size(hip, be, orc, ws):
    """72 x 72 grid, width 1024, 16 heads: 9 windows of 576 tokens (ws=24)
    or global attention over 5184 tokens (ws=0). The whole output, every
    row of every (window, head), against the oracle's attention region
    (LayerNorm, QKV projection, RoPE, the profile=cpu attention sequence):
    sam3_model.c:981-1013 end to end at the configs' full size."""
    grid, E, H = 72, 1024, 16
    x, n1w, n1b, w, b, table, want = _full_region_oracle(orc, ws)
    blk = hip.VitBlock()
    blk.n1w, blk.n1b = be.upload(n1w), be.upload(n1b)
    blk.qkvw, blk.qkvb = be.upload_weight(w), be.upload(b)
    blk.window = ws
    m = hip.Model(be, grid=grid, embed=E, heads=H, blocks=[blk])
    if ws:
        m.m.rope_win = be.upload(table)
    else:
        m.m.rope_glob = be.upload(table)
    be.write(m.m.x, 0, x)
    hip.vit_attention(m, blk)
    rows = want.shape[0]
    got = be.read(m.m.attn, rows * E).reshape(rows, E)
    m.free()
    assert report("attention region ws=%d %s (all %d rows)" % (ws, be.precision, rows),
                  got, want) <= TOL[be.precision]
    # Per (unit, head) as well: no block of the output may hide behind the
    # average over the whole.
    s = ws if ws else grid
    N = s * s
    worst = max(rel_l2(got[u * N:(u + 1) * N, h * 64:(h + 1) * 64],
                       want[u * N:(u + 1) * N, h * 64:(h + 1) * 64])
                for u in range(rows // N) for h in range(H))
    assert worst <= TOL[be.precision], worst


@pytest.mark.parametrize("grid,ws,E,H", [(16, 8, 128, 2), (24, 8, 128, 2), (16, 0, 128, 2),
                                         (72, 24, 1024, 16), (72, 0, 1024, 16)])
def test_packed_projection_matches_packing_kernel(hip, orc, grid, ws, E, H):
    """bf16 path: the operands the QKV projection's store packs (RoPE,
    scale, bf16, V^T, key block norms) are the packing kernel's, bit for
    bit (norm bounds to 1e-6), on the same device projection, at small
    shapes and at the full-size windowed and global blocks (projection
    tiles spanning windows, every unit and key block of a 72 x 72 grid)."""
    be = hip.Backend(precision="bf16")
    x, n1w, n1b, w, b = block_inputs(grid + 3 * ws, grid, E)
    s = ws if ws else grid
    N = s * s
    rows = (grid // s) ** 2 * N
    nb = rows // N * H
    table = orc.rope_table(s)
    blk = hip.VitBlock()
    blk.n1w, blk.n1b = be.upload(n1w), be.upload(n1b)
    blk.qkvw, blk.qkvb = be.upload_weight(w), be.upload(b)
    blk.window = ws
    m = hip.Model(be, grid=grid, embed=E, heads=H, blocks=[blk])
    tab = be.upload(table)
    if ws:
        m.m.rope_win = tab
    else:
        m.m.rope_glob = tab
    be.write(m.m.x, 0, x)
    hip.vit_attention(m, blk)
    fused = [be.read(getattr(m.m, k), nb * N * 64) for k in ("q16", "k16", "vt16")]
    kn_fused = be.read(m.m.knorm, nb * N // 64)
    hip.linear(m, rows, E, 3 * E, m.m.xn16, 0, blk.qkvw, blk.qkvb, m.m.qkv, 0)
    q = m.m.qkv
    hip.attn_fused(m, N, nb, H, hip.bmat(q, 0, 3 * E, N * 3 * E, 64),
                   hip.bmat(q, E, 3 * E, N * 3 * E, 64),
                   hip.bmat(q, 2 * E, 3 * E, N * 3 * E, 64),
                   hip.bmat(m.m.attn, 0, E, N * E, 64), tab, N, 0.125)
    kernel = [be.read(getattr(m.m, k), nb * N * 64) for k in ("q16", "k16", "vt16")]
    kn_kernel = be.read(m.m.knorm, nb * N // 64)
    m.free()
    be.free()
    for name, a, c in zip(("q16", "k16", "vt16"), fused, kernel):
        assert np.array_equal(a, c), name
    assert np.all(kn_fused > 0)
    assert rel_l2(kn_fused, kn_kernel) <= 1e-6
