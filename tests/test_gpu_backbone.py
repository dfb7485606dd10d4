"""GPU parity of the image encoder trunk against the oracle: whole ViT
blocks (vit_block, sam3_model.c:981-1028: attention region, projection
with residual / window_unpartition_add, norm2, erf-GELU MLP with residual)
and the trunk prologue (sam_encode_trunk, sam3_model.c:1112-1135: patch
im2col, patch GEMM, tiled position embedding, ln_pre).

Bars: rel-L2 <= 2e-5 on the fp32 path, <= 2e-2 on the bf16 path, on the
block's output tokens; max-abs printed with every check. Inputs are
random-init weights (tests/backbone_case.py) and N(0, 1) tokens.
"""
import numpy as np
import pytest

import backbone_case as bc
from gpu_common import report

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


def upload_block(hip, be, w):
    blk = hip.VitBlock()
    for k in ("n1w", "n1b", "qkvb", "projb", "n2w", "n2b", "l1b", "l2b"):
        setattr(blk, k, be.upload(w[k]))
    for k in ("qkvw", "projw", "l1w", "l2w"):
        setattr(blk, k, be.upload_weight(w[k]))
    blk.window = w["window"]
    return blk


def run_block(hip, be, orc, grid, E, heads, mlp, ws, seed, unfused=False):
    g = np.random.default_rng(seed)
    w = bc.block_weights(g, E, mlp, ws)
    x = g.standard_normal((grid * grid, E), dtype=np.float32)
    table = orc.rope_table(ws if ws else grid)
    blk = upload_block(hip, be, w)
    m = hip.Model(be, grid=grid, embed=E, heads=heads, blocks=[blk], mlp=mlp)
    if ws:
        m.m.rope_win = be.upload(table)
    else:
        m.m.rope_glob = be.upload(table)
    be.write(m.m.x, 0, x)
    print("vit_block grid=%d E=%d mlp=%d ws=%d unfused=%d %s" %
          (grid, E, mlp, ws, unfused, be.precision), flush=True)
    hip.vit_block(m, blk, unfused)
    got = be.read(m.m.x, grid * grid * E).reshape(grid * grid, E)
    m.free()
    want = orc.vit_block(x, grid, E, heads, 64, mlp, w, table)
    return got, want


@pytest.mark.parametrize("grid,ws", [(12, 6), (12, 0), (10, 4)])
@pytest.mark.parametrize("unfused", [False, True])
def test_vit_block_small(hip, be, orc, grid, ws, unfused):
    got, want = run_block(hip, be, orc, grid, 128, 2, 256, ws, 70 + grid + ws,
                          unfused)
    assert report("vit_block grid=%d ws=%d unfused=%d %s" %
                  (grid, ws, unfused, be.precision), got, want) <= TOL[be.precision]


@pytest.mark.parametrize("ws", [24, 0])
def test_vit_block_full_size(hip, be, orc, ws):
    """One block of the 72 x 72 x 1024 trunk, 16 heads, MLP 4096."""
    got, want = run_block(hip, be, orc, 72, 1024, 16, 4096, ws, 80 + ws)
    assert report("vit_block full ws=%d %s" % (ws, be.precision), got,
                  want) <= TOL[be.precision]


def trunk(hip, be, orc, grid, ps, E, heads, mlp, windows, seed, pe_f32=False):
    img, pe_w, pos, lnpw, lnpb, blocks = bc.trunk_case(seed, grid, ps, E, mlp,
                                                       windows)
    blks = [upload_block(hip, be, w) for w in blocks]
    wins = [w for w in windows if w]
    rw = orc.rope_table(wins[0]) if wins else None
    rg = orc.rope_table(grid)
    m = hip.Model(be, grid=grid, embed=E, heads=heads, blocks=blks, mlp=mlp)
    m.m.patch = ps
    m.m.pe_w = be.upload(pe_w) if pe_f32 else be.upload_weight(pe_w)
    m.m.pos, m.m.lnpw, m.m.lnpb = be.upload(pos), be.upload(lnpw), be.upload(lnpb)
    if rw is not None:
        m.m.rope_win = be.upload(rw)
    m.m.rope_glob = be.upload(rg)
    print("trunk grid=%d ps=%d E=%d depth=%d %s" %
          (grid, ps, E, len(windows), be.precision), flush=True)
    hip.sam_encode_trunk(m, img)
    be.finish()
    got = be.read(m.m.x, grid * grid * E).reshape(grid * grid, E)
    m.free()
    want = orc.encode_trunk(img, grid, ps, E, heads, 64, mlp, pe_w, pos, lnpw,
                            lnpb, blocks, rw, rg)
    return got, want


def test_encode_trunk_small(hip, be, orc):
    got, want = trunk(hip, be, orc, 8, 4, 128, 2, 256, [4, 0, 4], 90)
    assert report("trunk small %s" % be.precision, got,
                  want) <= TOL[be.precision]


def test_trunk_patch_weight_f32(hip, be, orc):
    """The patch weight left in float32 storage. With precision=bf16 the
    patch embedding pads the weight rows to whole 64-wide K steps and
    rounds them to bf16 in the same copy: the same bits as upload_weight's
    rounding, so the trunk's output equals the bf16-stored weight's run.
    With fp32 the exact path takes the float weight either way."""
    got, want = trunk(hip, be, orc, 8, 4, 128, 2, 256, [4, 0, 4], 92, pe_f32=True)
    assert report("trunk small, fp32 patch weight %s" % be.precision, got,
                  want) <= TOL[be.precision]
    ref, _ = trunk(hip, be, orc, 8, 4, 128, 2, 256, [4, 0, 4], 92)
    assert np.array_equal(got, ref)


def test_trunk_prologue_full_size(hip, be, orc):
    """Patch embedding of a 1008 x 1008 image (patch 14 -> 72 x 72 tokens
    of width 1024), position embedding and ln_pre, no blocks."""
    got, want = trunk(hip, be, orc, 72, 14, 1024, 16, 4096, [], 91)
    assert report("trunk prologue full %s" % be.precision, got,
                  want) <= TOL[be.precision]


# The 1008 x 1008 trunk: 32 blocks, global at 0-based 7, 15, 23, 31,
# 24 x 24 windows elsewhere (sam3_model.c:1112-1135, model.c:541-548).
FULL_WINDOWS = [0 if i in (7, 15, 23, 31) else 24 for i in range(32)]
_full_oracle = {}


def full_trunk_case():
    """Inputs of the full trunk and the oracle's output (computed once per
    session: the reference's profile=cpu sequence over 4.96 TFLOP)."""
    if "case" not in _full_oracle:
        from oracle import oracle as orc
        case = bc.trunk_case(97, 72, 14, 1024, 4096, FULL_WINDOWS, pt=24)
        img, pe_w, pos, lnpw, lnpb, blocks = case
        print("oracle: full trunk, 32 blocks", flush=True)
        want = orc.encode_trunk(img, 72, 14, 1024, 16, 64, 4096, pe_w, pos,
                                lnpw, lnpb, blocks, orc.rope_table(24),
                                orc.rope_table(72))
        print("oracle: done", flush=True)
        _full_oracle["case"] = (case, want)
    return _full_oracle["case"]


def test_trunk_full_size(hip, be, orc):
    """The whole image encoder trunk of a 1008 x 1008 image: patch 14 ->
    72 x 72 tokens of width 1024, 32 blocks of 16 heads x 64 with MLP
    4096, axial RoPE, position embedding tiled from the 24 x 24
    pretraining grid. The eager run against the oracle, then two replays
    of the captured trunk graph (another image between them) bit for bit
    against the eager run."""
    (img, pe_w, pos, lnpw, lnpb, blocks), want = full_trunk_case()
    grid, E = 72, 1024
    blks = [upload_block(hip, be, w) for w in blocks]
    m = hip.Model(be, grid=grid, embed=E, heads=16, blocks=blks, mlp=4096)
    m.m.patch = 14
    m.m.pe_w = be.upload_weight(pe_w)
    m.m.pos, m.m.lnpw, m.m.lnpb = be.upload(pos), be.upload(lnpw), be.upload(lnpb)
    m.m.rope_win = be.upload(orc.rope_table(24))
    m.m.rope_glob = be.upload(orc.rope_table(grid))
    try:
        def run(x):
            hip.sam_encode_trunk(m, x)
            be.finish()
            return be.read(m.m.x, grid * grid * E).reshape(grid * grid, E)

        print("trunk full 32 blocks %s: eager" % be.precision, flush=True)
        eager = run(img)
        assert np.isfinite(eager).all()
        assert report("trunk full %s" % be.precision, eager,
                      want) <= TOL[be.precision]
        other = np.ascontiguousarray(img[:, ::-1, :])
        print("trunk full 32 blocks %s: graph replays" % be.precision, flush=True)
        hip.sam_trunk_graph(m)
        assert m.m.trunk_exec
        first = run(img)
        flipped = run(other)
        again = run(img)
        assert np.array_equal(first, eager)
        assert np.array_equal(again, eager)
        assert not np.array_equal(flipped, eager)
        hip.sam_trunk_graph(m, False)
    finally:
        m.free()


def test_trunk_graph_replay(hip, be, orc):
    """HIP-graph replay of the trunk (sam_trunk_graph): every replay, with
    alternating images and eager work plus synchronisations between
    replays, equals the kernel-by-kernel run bit for bit; a later
    work-buffer reallocation drops the graph and the trunk still computes
    the same result; dropping the graph returns to the eager path."""
    grid, ps, E, heads, mlp, windows = 16, 4, 128, 2, 256, [8, 0, 8]
    img1, pe_w, pos, lnpw, lnpb, blocks = bc.trunk_case(95, grid, ps, E, mlp,
                                                        windows)
    img2 = bc.trunk_case(96, grid, ps, E, mlp, windows)[0]
    blks = [upload_block(hip, be, w) for w in blocks]
    m = hip.Model(be, grid=grid, embed=E, heads=heads, blocks=blks, mlp=mlp)
    m.m.patch = ps
    m.m.pe_w = be.upload_weight(pe_w)
    m.m.pos, m.m.lnpw, m.m.lnpb = be.upload(pos), be.upload(lnpw), be.upload(lnpb)
    m.m.rope_win = be.upload(orc.rope_table(8))
    m.m.rope_glob = be.upload(orc.rope_table(grid))
    print("trunk graph grid=%d %s" % (grid, be.precision), flush=True)

    def run(img):
        hip.sam_encode_trunk(m, img)
        be.finish()
        return be.read(m.m.x, grid * grid * E)

    eager = [run(img1), run(img2)]
    assert not np.array_equal(eager[0], eager[1])
    hip.sam_trunk_graph(m)
    assert m.m.trunk_exec
    other = be.upload(np.ones(4096, np.float32))
    for rep in range(4):
        got = run(img1 if rep % 2 == 0 else img2)
        assert np.array_equal(got, eager[rep % 2]), rep
        hip.add_bcast(m, other, other, other, 4096, 4096)
        be.finish()
    assert m.m.trunk_exec
    # Larger packed attention operands (bf16 path) reallocate work buffers.
    N = 1000
    qkv = be.upload(np.random.default_rng(1).standard_normal((N, 3 * E),
                                                             np.float32))
    out = be.alloc(N * E * 4)
    hip.attn_fused(m, N, heads, heads, hip.bmat(qkv, 0, 3 * E, 0, 64),
                   hip.bmat(qkv, E, 3 * E, 0, 64),
                   hip.bmat(qkv, 2 * E, 3 * E, 0, 64),
                   hip.bmat(out, 0, E, 0, 64), None, 1, 0.125)
    assert np.array_equal(run(img1), eager[0])
    if be.precision == "bf16":
        assert not m.m.trunk_exec
    hip.sam_trunk_graph(m, False)
    assert not m.m.trunk_exec
    assert np.array_equal(run(img2), eager[1])
    be.release(qkv)
    be.release(out)
    be.release(other)
    m.free()
