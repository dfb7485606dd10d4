"""Attention-path benchmark on one MI355X.

Step = one pass of the fused attention of a global ViT block: 5184 tokens
(72 x 72 grid), 16 heads of 64, 2D RoPE, bf16 MFMA with f32 accumulation,
operands resident in HBM (packed by the block's LayerNorm -> QKV
projection -> packing, which run before the timed region). `value` is
attention TFLOP/s = 4 * 5184^2 * 64 * 16 FLOP per step / step time; the
same JSON line reports the 9 x 576 windowed batch, the fp32 exact path,
the QKV projection GEMM, the whole attention region, the mask-decoder
cross-attention (GB/s), the dominant kernel's roofline and the CPU
baseline (the oracle's restatement of the reference's profile=cpu
sequence on the host cores).

Order: the host-side sections run first, then the GPU sections (fp32
path, decoder, mask decoder, text path, backbone), then ~27 ms of the
global attention region back to back (COND_REGIONS), then the headline's
W warm-up and K timed launches, so that those K launches (a few ms at
most) see the engine clock at its loaded steady state instead of its
ramp from idle (from idle the clock needs 10-20 ms of sustained work);
the windowed line follows the same protocol with its own block's
region, and the single window (bf16, then fp32) right after it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import importlib.util
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "i.sam3.opencl_amd")

METRIC = ("attention TFLOP/s + % MFMA peak (5184-tok global, 9×576 "
          "window); backbone ms/img")
PEAK_BF16 = 2516.6   # TFLOP/s, dense bf16 MFMA, MI355X
PEAK_F32 = 157.3     # TFLOP/s, f32 MFMA
PEAK_HBM = 8000.0    # GB/s
COPY_BYTES = 256 << 20
# Replays of a block's attention region (LayerNorm, QKV projection,
# attention; ~0.18 ms global, ~0.08 ms windowed) that bring the engine
# clock to its loaded state before a line's warm-up steps: the headline
# (global) and the windowed line are each conditioned by their own block.
COND_REGIONS = 150

# HBM bytes per k_attn_bf16 launch (global, 5184 tokens x 16 heads), from
# rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of `bench.py --kernel-only`
# (KiB per dispatch, mean of 5), each scaled by what the counter reads for
# the same run's LayerNorm, whose bytes are known exactly (5184 x 1024 fp32
# read with gamma and beta, 20744 KiB, against FETCH_SIZE 10470 KiB; 5184 x
# 1024 bf16 written, 10368 KiB, against WRITE_SIZE 10368 KiB). Above the
# operands and O (15650 / 20740 KiB on the plain grid), the balanced
# launch's piece records of cut tiles, stored and read back with
# agent-scope atomics, add ~11 MB fetched and ~16 MB written. Summary and
# commands: profiles/attn_bf16_global_5184.md.
ATTN_FETCH_KIB, ATTN_WRITE_KIB = 21110.0, 36880.0
FETCH_SCALE, WRITE_SCALE = 20744.0 / 10470.0, 10368.0 / 10368.0


def load_hip():
    spec = importlib.util.spec_from_file_location(
        "sam3_hip", os.path.join(PKG, "sam3_hip.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["sam3_hip"] = mod
    spec.loader.exec_module(mod)
    mod.lib()
    return mod


def rope_table(side, hd=64, theta=10000.0):
    """Axial 2D RoPE (cos, sin) table: pair k < 16 rotates by x * f_k,
    pair 16 + k by y * f_k, f_k = theta^(-4k/64), position y * side + x."""
    f = theta ** (-4.0 * np.arange(hd // 4) / hd)
    pos = np.arange(side * side)
    ang = np.concatenate([np.outer(pos % side, f), np.outer(pos // side, f)], 1)
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)


def block_inputs(seed, grid=72, E=1024):
    g = np.random.default_rng(seed)
    x = g.standard_normal((grid * grid, E), dtype=np.float32)
    bound = math.sqrt(6.0 / (E + 3 * E))
    w = g.uniform(-bound, bound, (3 * E, E)).astype(np.float32)
    b = g.uniform(-1 / math.sqrt(E), 1 / math.sqrt(E), 3 * E).astype(np.float32)
    return x, w, b


class Block:
    """One ViT block's attention region on the device (random init)."""

    def __init__(self, hip, be, ws, seed, grid=72, E=1024, H=16):
        self.hip, self.be, self.ws, self.E, self.H = hip, be, ws, E, H
        x, w, b = block_inputs(seed, grid, E)
        s = ws if ws else grid
        self.N = s * s
        self.nunits = ((grid + s - 1) // s) ** 2
        blk = hip.VitBlock()
        blk.n1w = be.upload(np.ones(E, np.float32))
        blk.n1b = be.upload(np.zeros(E, np.float32))
        blk.qkvw = be.upload_weight(w)
        blk.qkvb = be.upload(b)
        blk.window = ws
        self.blk = blk
        self.m = hip.Model(be, grid=grid, embed=E, heads=H, blocks=[blk])
        tab = be.upload(rope_table(s))
        if ws:
            self.m.m.rope_win = tab
        else:
            self.m.m.rope_glob = tab
        be.write(self.m.m.x, 0, x)
        self.rows = self.nunits * self.N
        self.out = hip.bmat(self.m.m.attn, 0, E, self.N * E, 64)

    def flops(self):
        return 4.0 * self.N * self.N * 64 * self.H * self.nunits

    def bytes(self):
        """Algorithmic bytes of the packed-operand kernel: bf16 Q, K, V^T
        read once, fp32 O written once."""
        units = self.nunits * self.H
        return units * self.N * 64 * (3 * 2 + 4)

    def region(self):
        self.hip.vit_attention(self.m, self.blk)

    def attn(self):
        """The attention kernel alone on the packed operands."""
        self.hip.attn_packed(self.m, self.N, self.nunits * self.H, self.H,
                             self.out)

    def attn_f32(self):
        E, N = self.E, self.N
        q = self.m.m.qkv
        tab = self.m.m.rope_win if self.ws else self.m.m.rope_glob
        self.hip.attn_fused(self.m, N, self.nunits * self.H, self.H,
                            self.hip.bmat(q, 0, 3 * E, N * 3 * E, 64),
                            self.hip.bmat(q, E, 3 * E, N * 3 * E, 64),
                            self.hip.bmat(q, 2 * E, 3 * E, N * 3 * E, 64),
                            self.out, tab, N, 0.125)

    def qkv_gemm(self):
        E = self.E
        src = self.m.m.xn16 if self.m.m.xn16 else self.m.m.xn
        self.hip.linear(self.m, self.rows, E, 3 * E, src, 0, self.blk.qkvw,
                        self.blk.qkvb, self.m.m.qkv, 0, 0, 0)


def timed(be, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    be.finish()
    be.timer_start()
    for _ in range(steps):
        fn()
    ms = be.timer_stop()
    return ms / steps


def bf16_bits(x):
    """fp32 -> bf16 storage bits, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)


# The trunk's four GEMM shapes at 72 x 72 tokens (sam_encode_trunk):
# (rows, in, out, activation, residual add, bf16 output).
TRUNK_GEMMS = {"qkv": (5184, 1024, 3072, 0, 0, False),
               "proj": (5184, 1024, 1024, 0, 1, False),
               "fc1": (5184, 1024, 4096, 1, 0, True),
               "fc2": (5184, 4096, 1024, 0, 1, False)}


def trunk_gemms(hip, steps, warmup, rounds=5):
    """The trunk's GEMMs through linear() (bf16 operands, fp32 accumulate,
    the trunk's epilogue: bias, GELU on fc1 with a bf16 store, residual
    add on the projection and fc2) beside the platform's hipBLASLt
    (torch.nn.functional.linear, bias only, bf16 out) on the same
    N(0, 1) operands. The engine clock under MFMA load depends on the
    data, so both legs see the same random values. Median of `rounds`
    event-timed runs of `steps` launches each."""
    import torch
    torch.cuda.init()     # the shared runtime, initialised through torch first
    be = hip.Backend(precision="bf16")
    m = hip.Model(be, embed=128, heads=2)
    g = np.random.default_rng(0)
    out = {}
    for name, (M, K, N, act, res, cbf) in TRUNK_GEMMS.items():
        a16 = bf16_bits(g.standard_normal((M, K), dtype=np.float32))
        w16 = bf16_bits(g.standard_normal((N, K), dtype=np.float32))
        bias = g.standard_normal(N, dtype=np.float32)
        A = be.upload_typed(a16, hip.BF16)
        W = be.upload_typed(w16, hip.BF16)
        B = be.upload(bias)
        c0 = g.standard_normal((M, N), dtype=np.float32)
        C = be.upload_typed(bf16_bits(c0), hip.BF16) if cbf else be.upload(c0)

        def lib_call():
            hip.linear(m, M, K, N, A, 0, W, B, C, 0, act, res)

        fl = 2.0 * M * N * K
        lib_ms = sorted(timed(be, lib_call, steps, warmup)
                        for _ in range(rounds))[rounds // 2]
        for d in (A, W, B, C):
            be.release(d)
        ta = torch.from_numpy(a16.view(np.int16)).view(torch.bfloat16).cuda()
        tw = torch.from_numpy(w16.view(np.int16)).view(torch.bfloat16).cuda()
        tb = torch.from_numpy(bias).cuda().bfloat16()

        def torch_call():
            torch.nn.functional.linear(ta, tw, tb)

        ts = []
        for _ in range(rounds):
            for _ in range(warmup):
                torch_call()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                torch_call()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) / steps)
        t_ms = sorted(ts)[rounds // 2]
        del ta, tw, tb
        out[name] = {"shape": [M, K, N], "us": round(1e3 * lib_ms, 2),
                     "TFLOP/s": round(fl / lib_ms / 1e9, 1),
                     "hipblaslt_us": round(1e3 * t_ms, 2),
                     "hipblaslt_TFLOP/s": round(fl / t_ms / 1e9, 1)}
    m.free()
    be.free()
    return out


def backbone_flops(grid=72, E=1024, mlp=4096, ps=14, depth=32, ws=24,
                   glob_at=(7, 15, 23, 31)):
    """Algorithmic FLOPs of one image through the trunk: patch GEMM, per
    block QKV / projection / MLP GEMMs and attention (4 N^2 64 per window
    and head)."""
    T = grid * grid
    f = 2.0 * T * 3 * ps * ps * E
    for i in range(depth):
        s = grid if i in glob_at else ws
        nwin = (-(-grid // s)) ** 2
        f += 2.0 * T * E * (3 * E + E + 2 * mlp)
        f += 4.0 * (s * s) ** 2 * 64 * (E // 64) * nwin
    return f


def backbone(hip, steps, warmup, precisions=("bf16", "fp32")):
    """Image encoder trunk, end to end (sam_encode_trunk): 1008 x 1008 x 3
    image ~ U(0, 1) normalised (x - 0.5) / 0.5, patch 14 -> 72 x 72 tokens
    of width 1024, 32 blocks (global attention at blocks 7, 15, 23, 31,
    24 x 24 windows elsewhere), 16 heads x 64, MLP 4096 erf-GELU, 2D RoPE;
    random-init weights (Xavier-uniform linears, U(+-1/sqrt(fan_in))
    biases, LayerNorm 1 / 0, position embedding tiled from a 24 x 24
    grid). ms per image for precision=bf16 and =fp32, and the attention
    kernels' share of a pass whose launches are timed in flow."""
    grid, E, H, mlp, ps, depth = 72, 1024, 16, 4096, 14, 32
    glob_at = (7, 15, 23, 31)
    g = np.random.default_rng(17)

    def xavier(o, i):
        b = math.sqrt(6.0 / (i + o))
        return (g.random((o, i), dtype=np.float32) * (2 * b) - b)

    def bias(n, fan):
        b = 1.0 / math.sqrt(fan)
        return (g.random(n, dtype=np.float32) * (2 * b) - b)

    bes = {p: hip.Backend(precision=p) for p in precisions}
    blocks = {p: [] for p in bes}
    ones, zeros = np.ones(E, np.float32), np.zeros(E, np.float32)
    for i in range(depth):
        w = {"qkvw": xavier(3 * E, E), "qkvb": bias(3 * E, E),
             "projw": xavier(E, E), "projb": bias(E, E),
             "l1w": xavier(mlp, E), "l1b": bias(mlp, E),
             "l2w": xavier(E, mlp), "l2b": bias(E, mlp)}
        for p, be in bes.items():
            blk = hip.VitBlock()
            for k in ("qkvw", "projw", "l1w", "l2w"):
                setattr(blk, k, be.upload_weight(w[k]))
            for k in ("qkvb", "projb", "l1b", "l2b"):
                setattr(blk, k, be.upload(w[k]))
            blk.n1w, blk.n2w = be.upload(ones), be.upload(ones)
            blk.n1b, blk.n2b = be.upload(zeros), be.upload(zeros)
            blk.window = 0 if i in glob_at else 24
            blocks[p].append(blk)
    pe_w = xavier(E, 3 * ps * ps)
    pe = (0.02 * g.standard_normal((24 * 24, E))).astype(np.float32)
    yy, xx = np.divmod(np.arange(grid * grid), grid)
    pos = np.ascontiguousarray(pe[(yy % 24) * 24 + xx % 24])
    side = grid * ps
    img = ((g.random((3, side, side), dtype=np.float32) - 0.5) / 0.5)
    out = {"workload": "image encoder trunk: 1008x1008x3 image, patch 14 -> "
                       "72x72 tokens x 1024, 32 blocks (global at 7/15/23/31, "
                       "24x24 windows), 16 heads x 64, MLP 4096, 2D RoPE",
           "tflop_per_img": round(backbone_flops() / 1e12, 3)}
    for p, be in bes.items():
        m = hip.Model(be, grid=grid, embed=E, heads=H, blocks=blocks[p],
                      mlp=mlp)
        m.m.patch = ps
        m.m.pe_w = be.upload_weight(pe_w)
        m.m.pos, m.m.lnpw, m.m.lnpb = be.upload(pos), be.upload(ones), be.upload(zeros)
        m.m.rope_win = be.upload(rope_table(24))
        m.m.rope_glob = be.upload(rope_table(grid))
        ms_eager = timed(be, lambda: hip.sam_encode_trunk(m, img), steps,
                         warmup)
        # The same trunk replayed from a HIP graph (one launch per image
        # after the image upload).
        hip.sam_trunk_graph(m)
        ms = timed(be, lambda: hip.sam_encode_trunk(m, img), steps, warmup)
        # One pass with every launch bracketed by events in flow (profile
        # 2: no wait between launches, as in the eager run) for the
        # per-kernel times and the attention share.
        hip.prof_reset()
        be._b.profile = 2
        hip.sam_encode_trunk(m, img)
        be.finish()
        be._b.profile = 0
        tab = hip.prof_table()
        tot = sum(r[1] for r in tab)
        att = sum(r[1] for r in tab if r[0] in ("attn_bf16", "qkv_pack",
                                                "attn_f32"))
        hip.sam_trunk_graph(m, False)
        out[p] = {"ms_per_img": round(ms, 3),
                  "ms_per_img_kernel_by_kernel": round(ms_eager, 3),
                  "TFLOP/s": round(backbone_flops() / ms / 1e9, 1),
                  "attention_share": round(att / tot, 4),
                  "profile_ms": {r[0]: round(r[1], 3) for r in
                                 sorted(tab, key=lambda r: -r[1])[:8]}}
        m.free()
    for be in bes.values():
        be.free()
    return out


def text_attention(hip, steps, warmup):
    """The text path's attend() (sam3_text.c:305-343) at its two large
    shapes, random N(0, 1) operands: the fusion encoder's self-attention
    over the 72 x 72 image tokens (8 heads x 32, no mask: the fused kernel
    on bf16, the reference's chunked gemm / softmax_ext / gemm on fp32) and
    the decoder's cross-attention of 201 queries to the image with the box
    relative position bias (gemm / softmax_ext / gemm). TFLOP/s counts
    4 Nq Nk hd per head."""
    out = {}
    g = np.random.default_rng(41)
    heads, hd, N, W, Nq = 8, 32, 5184, 72, 201
    D = heads * hd
    for p in ("bf16", "fp32"):
        be = hip.Backend(precision=p)
        m = hip.Model(be, embed=128, heads=2)
        q, k, v = (be.upload(g.standard_normal((N, D), dtype=np.float32))
                   for _ in range(3))
        o = be.alloc(N * D * 4)
        dy = be.upload(g.standard_normal((Nq, W, heads), dtype=np.float32))
        dx = be.upload(g.standard_normal((Nq, W, heads), dtype=np.float32))
        st, wu = (steps, warmup) if p == "bf16" else (max(2, steps // 20), 1)
        ms = timed(be, lambda: hip.attend(m, N, N, heads, hd, q, D, k, D, v, D,
                                          o, D), st, wu)
        ms_box = timed(be, lambda: hip.attend(m, Nq, N, heads, hd, q, D, k, D,
                                              v, D, o, D, False, dy, dx, W),
                       max(2, steps // 10), max(1, warmup // 10))
        out["fusion_self_" + p] = {
            "workload": "5184 tokens, 8 heads x 32, no mask",
            "ms": round(ms, 4),
            "TFLOP/s": round(4.0 * N * N * hd * heads / ms / 1e9, 1)}
        out["decoder_box_" + p] = {
            "workload": "201 queries x 5184 keys, 8 heads x 32, box bias",
            "ms": round(ms_box, 4),
            "TFLOP/s": round(4.0 * Nq * N * hd * heads / ms_box / 1e9, 2)}
        for d in (q, k, v, o, dy, dx):
            be.release(d)
        m.free()
        be.free()
    return out


def cpu_baseline(steps=3):
    """The oracle's restatement of the reference's profile=cpu attention of
    the global block (gemm_cpu_t Q K^T with alpha 1/8 -> softmax_rows ->
    gemm_cpu_n P V, 4 heads per score-buffer chunk), timed on the host
    cores; median of `steps` after one warm-up."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc

    N, H, E, hc = 5184, 16, 1024, 4
    g = np.random.default_rng(5)
    qkv = g.standard_normal((N, 3 * E), dtype=np.float32)
    out = np.zeros((N, E), np.float32)
    S = np.zeros((hc, N, N), np.float32)
    lib = orc.lib()

    def one():
        for h0 in range(0, H, hc):
            orc.gemm(orc.GEMM_CPU_T, N, N, 64, qkv, h0 * 64, 3 * E, 0, 64, qkv,
                     E + h0 * 64, 3 * E, 0, 64, 1, S, 0, N, 0, N * N, hc, hc,
                     alpha=0.125)
            lib.or_softmax_rows(S.ctypes.data, hc * N, N)
            orc.gemm(orc.GEMM_SEQ, N, 64, N, S, 0, N, 0, N * N, qkv,
                     2 * E + h0 * 64, 3 * E, 0, 64, 0, out, h0 * 64, E, 0, 64,
                     hc, hc)

    one()
    times = []
    for _ in range(steps):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    sec = float(np.median(times))
    return {"value": round(4.0 * N * N * 64 * H / sec / 1e12, 5),
            "unit": "TFLOP/s", "cores": orc.threads(), "kind": "port",
            "sample": "full 5184-token global attention, 16 heads x 64, "
                      "fp32, reference profile=cpu sequence restated in C "
                      "(median of %d, %.2f s each)" % (steps, sec)}


def cpu_configs():
    """The oracle's restatement of the reference's profile=cpu dispatch at
    the other workloads, on the host cores (one run each, after the
    headline's CPU baseline warmed the library): config 1 (one 576-token
    window, 16 heads), config 2 (the 9 x 576 windowed batch's attention),
    config 4 (the decoder cross-attention, P = 64, both directions) and
    config 5 (the whole 32-block trunk of a 1008 x 1008 image)."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import backbone_case as bc

    out = {}
    g = np.random.default_rng(6)
    E, H = 1024, 16
    for name, nunits in (("config1_window", 1), ("config2_windowed", 9)):
        N = 576
        qkv = g.standard_normal((nunits * N, 3 * E), dtype=np.float32)
        o = np.zeros((nunits * N, E), np.float32)
        S = np.zeros((nunits * H, N, N), np.float32)
        t0 = time.perf_counter()
        orc.gemm(orc.GEMM_CPU_T, N, N, 64, qkv, 0, 3 * E, N * 3 * E, 64, qkv, E,
                 3 * E, N * 3 * E, 64, 1, S, 0, N, H * N * N, N * N, nunits * H,
                 H, alpha=0.125)
        orc.lib().or_softmax_rows(S.ctypes.data, nunits * H * N, N)
        orc.gemm(orc.GEMM_SEQ, N, 64, N, S, 0, N, H * N * N, N * N, qkv, 2 * E,
                 3 * E, N * 3 * E, 64, 0, o, 0, E, N * E, 64, nunits * H, H)
        sec = time.perf_counter() - t0
        out[name] = {"ms": round(sec * 1e3, 1),
                     "GFLOP/s": round(4.0 * N * N * 64 * H * nunits / sec / 1e9, 1)}
    P, T, dint = 64, 4096, 128
    tok = g.standard_normal((P, 7, dint), dtype=np.float32)
    img = g.standard_normal((P, T, dint), dtype=np.float32)
    t0 = time.perf_counter()
    orc.mha(P, 7, T, dint, tok, 7 * dint, img, T * dint, img, T * dint)
    orc.mha(P, T, 7, dint, img, T * dint, tok, 7 * dint, tok, 7 * dint)
    sec = time.perf_counter() - t0
    out["config4_decoder"] = {"ms": round(sec * 1e3, 1),
                              "GB/s": round(2 * 268.9e6 / sec / 1e9, 2)}
    wins = [0 if i in (7, 15, 23, 31) else 24 for i in range(32)]
    img, pe_w, pos, lnpw, lnpb, blocks = bc.trunk_case(7, 72, 14, 1024, 4096,
                                                       wins, pt=24)
    t0 = time.perf_counter()
    orc.encode_trunk(img, 72, 14, 1024, 16, 64, 4096, pe_w, pos, lnpw, lnpb,
                     blocks, orc.rope_table(24), orc.rope_table(72))
    sec = time.perf_counter() - t0
    out["config5_backbone"] = {"ms_per_img": round(sec * 1e3, 1),
                               "TFLOP/s": round(backbone_flops() / sec / 1e12, 4)}
    out["cores"] = orc.threads()
    out["kind"] = "port"
    return out


def decoder(hip, be, steps, warmup):
    """Mask-decoder cross-attention, 64 prompts, per-prompt image keys
    (layer >= 1 semantics): token->image (7 x 4096 keys) and
    image->token (4096 queries x 7 keys), 8 heads x 16, fp32; GB/s of the
    algorithmic bytes (Q, K, V read once, O written once)."""
    P, T, NT, dint = 64, 4096, 7, 128
    m = hip.Model(be, embed=128, heads=2)
    g = np.random.default_rng(3)
    img = be.upload(g.standard_normal((P * T, dint), dtype=np.float32))
    img2 = be.upload(g.standard_normal((P * T, dint), dtype=np.float32))
    tok = be.upload(g.standard_normal((P * NT, dint), dtype=np.float32))
    tok2 = be.upload(g.standard_normal((P * NT, dint), dtype=np.float32))
    o_t = be.alloc(P * NT * dint * 4)
    o_i = be.alloc(P * T * dint * 4)
    t2i = timed(be, lambda: hip.mha(m, P, NT, T, dint, tok, NT * dint, img,
                                    T * dint, img2, T * dint, o_t), steps, warmup)
    i2t = timed(be, lambda: hip.mha(m, P, T, NT, dint, img, T * dint, tok,
                                    NT * dint, tok2, NT * dint, o_i), steps, warmup)
    # Practical HBM ceiling: the runtime's device-to-device copy of
    # COPY_BYTES (read + write).
    src = be.alloc(COPY_BYTES, "copy src")
    dst = be.alloc(COPY_BYTES, "copy dst")
    cp = timed(be, lambda: be.copy(src, dst, 0, 0, COPY_BYTES), steps, warmup)
    be.release(src)
    be.release(dst)
    bytes_t2i = 4.0 * (P * NT * dint * 2 + 2 * P * T * dint)
    bytes_i2t = 4.0 * (2 * P * T * dint + 2 * P * NT * dint)
    for d in (img, img2, tok, tok2, o_t, o_i):
        be.release(d)
    return {
        "t2i_ms": round(t2i, 4), "t2i_GBps": round(bytes_t2i / t2i / 1e6, 1),
        "i2t_ms": round(i2t, 4), "i2t_GBps": round(bytes_i2t / i2t / 1e6, 1),
        "pct_hbm_peak": round(100 * (bytes_t2i + bytes_i2t) / (t2i + i2t) /
                              1e6 / PEAK_HBM, 1),
        "device_copy_GBps": round(2.0 * COPY_BYTES / cp / 1e6, 1),
    }


def mask_decoder(hip, steps, warmup, precisions=("bf16", "fp32"), P=64,
                 grid=72):
    """The point-prompt mask decoder, sam_decode (sam3_model.c:1239-1400),
    P prompts on the 72 x 72 image embedding: prompt tokens, the two-way
    transformer with per-prompt image keys [P][5184][256], the output
    upscaling to [P][288][288][32], the host hypernetwork / IoU heads and
    the low-resolution logits [P][3][288][288]; random-init weights, image
    features ~ N(0, 1). ms per call of P prompts, and the per-operator
    profile of one pass."""
    g = np.random.default_rng(29)
    T = grid * grid
    w = hip.random_decoder_weights(29)
    emb = g.standard_normal((T, 256), dtype=np.float32)
    s0 = g.standard_normal((16 * T, 32), dtype=np.float32)
    s1 = g.standard_normal((4 * T, 64), dtype=np.float32)
    pts = g.uniform(0, 14 * grid, (P, 2)).astype(np.float32)
    out = {"workload": "sam_decode: %d single-point prompts, 72x72x256 image "
                       "embedding, per-prompt keys, upscaling to 288x288, "
                       "3 multimask logits" % P}
    for p in precisions:
        be = hip.Backend(precision=p)
        m = hip.Model(be, embed=1024, heads=16)
        m.m.grid = grid
        dec = hip.Decoder(m, w, P, img=14 * grid)
        dec.set_image(emb, s0, s1)
        ms_eager = timed(be, lambda: dec.decode(pts), steps, warmup)
        # The device sequence replayed from a HIP graph (one launch after
        # the token upload).
        dec.graph(P)
        ms = timed(be, lambda: dec.decode(pts), steps, warmup)
        dec.graph(P, False)
        hip.prof_reset()
        be._b.profile = 2
        dec.decode(pts)
        be.finish()
        be._b.profile = 0
        tab = hip.prof_table()
        out[p] = {"ms": round(ms, 3), "ms_kernel_by_kernel": round(ms_eager, 3),
                  "profile_ms": {r[0]: round(r[1], 3) for r in
                                 sorted(tab, key=lambda r: -r[1])[:10]}}
        dec.free()
        m.free()
        be.free()
    return out


def mask_decoder_cpu(P=2, grid=72):
    """The oracle's restatement of sam_decode (fp32, the reference's GPU
    dispatch arithmetic, OpenMP over the host cores) for P prompts on the
    same synthetic inputs: seconds per prompt, for scale against the
    64-prompt GPU figure."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    hip = load_hip()
    g = np.random.default_rng(29)
    T = grid * grid
    w = hip.random_decoder_weights(29)
    emb = g.standard_normal((T, 256), dtype=np.float32)
    s0 = g.standard_normal((16 * T, 32), dtype=np.float32)
    s1 = g.standard_normal((4 * T, 64), dtype=np.float32)
    pts = g.uniform(0, 14 * grid, (P, 2)).astype(np.float32)
    dw = orc.DecoderW(w, grid, img=14 * grid)
    prep = orc.dec_prepare(dw, emb)
    t0 = time.perf_counter()
    orc.sam_decode(dw, pts, prep, s0, s1)
    sec = time.perf_counter() - t0
    return {"ms_per_prompt": round(1e3 * sec / P, 2), "cores": orc.threads(),
            "kind": "port", "sample": "%d prompts, fp32, oracle restatement"
                                      % P}


def checkpoint_load(hip, precisions=("bf16", "fp32"), depth=8, reps=3):
    """Checkpoint weights into HBM. A SAM 3-named float32 checkpoint of
    the trunk's first `depth` blocks at their real shapes (E 1024, MLP
    4736, 16 heads; blocks 0-6 windowed 24 x 24, block 7 global 72 x 72
    with their complex64 rope tables; patch embedding, 24 x 24 + 1
    position embedding, ln_pre) and the point decoder, random values,
    written by torch.save to a temporary file that is read once before
    timing (page cache warm: memory -> HBM, not disk). Per precision:
    - upload: every tensor of the file by pth_upload into the element
      type the model keeps (weight matrices bf16 / f32, the rest f32),
      GB/s of file storage bytes;
    - reference_path: the reference's sequence for the same tensors
      (pth_read_f32 to host floats, host rounding of weight matrices,
      upload; sam3_model.c:52-76);
    - sam_load: the whole sam_load (weights, tiled position embedding,
      work buffers, decoder set-up for 64 prompts), ms."""
    import ctypes
    import tempfile
    import torch
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import pth_case as pc

    g = np.random.default_rng(41)
    E, M = 1024, 4736

    def rnd(*shape):
        return (0.02 * g.standard_normal(shape, dtype=np.float32))

    win = [24] * (depth - 1) + [0]
    blocks = [{"n1w": rnd(E), "n1b": rnd(E), "qkvw": rnd(3 * E, E),
               "qkvb": rnd(3 * E), "projw": rnd(E, E), "projb": rnd(E),
               "n2w": rnd(E), "n2b": rnd(E), "l1w": rnd(M, E), "l1b": rnd(M),
               "l2w": rnd(E, M), "l2b": rnd(E), "window": w} for w in win]
    ropes = [rope_table(w if w else 72) for w in win]
    tw = dict(E=E, patch=14, pe_w=rnd(E, 3 * 14 * 14),
              pos_embed=rnd(1, 577, E), lnpw=rnd(E), lnpb=rnd(E),
              blocks=blocks, ropes=ropes)
    sd = pc.sam3_names(tw, hip.random_decoder_weights(41))
    tmp = tempfile.mkdtemp(prefix="sam3ck_")
    path = os.path.join(tmp, "sam3_part.pt")
    pc.save_torch(path, sd)
    with open(path, "rb") as f:
        while f.read(1 << 26):
            pass
    nbytes = os.path.getsize(path)
    mats = {k for k, a in sd.items() if a.ndim >= 2 and "freqs" not in k and
            "pos_embed" not in k and "prompt_encoder" not in k and
            "_token" not in k and "tokens" not in k}
    out = {"workload": "SAM 3 checkpoint, trunk blocks 0-%d + point decoder, "
                       "float32 storage, %d tensors, %.0f MB" %
                       (depth - 1, len(sd), nbytes / 1e6)}
    ck = hip.Checkpoint(path)
    L = hip.lib()
    store = ck.bytes("")
    try:
        for p in precisions:
            be = hip.Backend(precision=p)
            wdt = hip.BF16 if p == "bf16" else hip.F32

            def upload():
                mems = []
                for k in sd:
                    dt = wdt if k in mats else hip.F32
                    mems.append(ck.upload(be, k, dt))
                be.finish()
                return mems

            def reference_path():
                mems = []
                for k in sd:
                    t = ck.find(k)
                    if t.dtype == hip.PTH_C64:
                        ptr = L.pth_read_c64(ck.ptr, ctypes.byref(t))
                        n = 2 * ck.numel(t)
                    else:
                        ptr = L.pth_read_f32(ck.ptr, ctypes.byref(t))
                        n = ck.numel(t)
                    if k in mats:
                        m = L.hipb_upload_weight(be.ptr, ptr, n, k.encode())
                    else:
                        m = L.hipb_upload(be.ptr, ptr, 4 * n, k.encode())
                    hip._libc.free(ptr)
                    mems.append(m)
                be.finish()
                return mems

            res = {}
            for name, fn in (("upload", upload),
                             ("reference_path", reference_path)):
                best = None
                for _ in range(reps):
                    t0 = time.perf_counter()
                    mems = fn()
                    dt_s = time.perf_counter() - t0
                    for mm in mems:
                        be.release(mm)
                    best = dt_s if best is None else min(best, dt_s)
                res[name] = {"ms": round(1e3 * best, 1),
                             "GB/s": round(store / best / 1e9, 2)}
            best = None
            for _ in range(reps):
                t0 = time.perf_counter()
                m = hip.Model.load(be, ck, batch=64, point_head=True)
                be.finish()
                dt_s = time.perf_counter() - t0
                m.free()
                best = dt_s if best is None else min(best, dt_s)
            res["sam_load_ms"] = round(1e3 * best, 1)
            res["speedup_vs_reference_path"] = round(
                res["reference_path"]["ms"] / res["upload"]["ms"], 2)
            out[p] = res
            be.free()
    finally:
        ck.close()
        os.remove(path)
        os.rmdir(tmp)
    out["storage_bytes"] = int(store)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # Enough untimed launches (about 30 ms) for the engine clock to settle.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only the global bf16 attention kernel (profiling)")
    ap.add_argument("--decoder-only", action="store_true",
                    help="only the mask-decoder cross-attention (profiling)")
    ap.add_argument("--mask-decoder-only", action="store_true",
                    help="only sam_decode of 64 prompts (profiling)")
    ap.add_argument("--backbone-only", action="store_true",
                    help="only the image encoder trunk (profiling)")
    ap.add_argument("--text-only", action="store_true",
                    help="only the text path's attend() shapes (profiling)")
    ap.add_argument("--one-window-only", action="store_true",
                    help="only the single 576-token window's attention, bf16 and "
                         "fp32 (profiling)")
    ap.add_argument("--window-only", action="store_true",
                    help="only the windowed bf16 attention kernel (profiling)")
    ap.add_argument("--region-only", action="store_true",
                    help="only the global block's attention region: LayerNorm, "
                         "packed QKV projection GEMM, attention (profiling)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the trunk's GEMM shapes beside hipBLASLt")
    ap.add_argument("--checkpoint-only", action="store_true",
                    help="only the checkpoint upload timings")
    ap.add_argument("--precision", choices=("bf16", "fp32"),
                    help="with --backbone-only: that path alone")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the attention path shards by image "
              "or crop (data parallel, no exchange between GPUs), so a "
              "multi-GPU figure is N independent copies of this one. Run "
              "with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.gemm_only:
        # torch before the library: the library's libamdhip64.so.7 then
        # binds to the runtime torch loaded (one HIP runtime per process).
        import torch  # noqa: F401
    hip = load_hip()
    if args.backbone_only:
        prec = (args.precision,) if args.precision else ("bf16", "fp32")
        print(json.dumps({"backbone": backbone(hip, args.steps, args.warmup,
                                               prec)}))
        return
    if args.mask_decoder_only:
        prec = (args.precision,) if args.precision else ("bf16", "fp32")
        print(json.dumps({"mask_decoder": mask_decoder(
            hip, args.steps, min(args.warmup, 5), prec)}))
        return
    if args.gemm_only:
        print(json.dumps({"trunk_gemms": trunk_gemms(
            hip, min(args.steps, 20), min(args.warmup, 30))}))
        return
    if args.checkpoint_only:
        prec = (args.precision,) if args.precision else ("bf16", "fp32")
        print(json.dumps({"checkpoint": checkpoint_load(hip, prec)}))
        return
    if args.text_only:
        print(json.dumps({"text_attention": text_attention(
            hip, args.steps, min(args.warmup, 20))}))
        return
    if args.decoder_only:
        be32 = hip.Backend(precision="fp32")
        print(json.dumps({"decoder_fp32": decoder(hip, be32, args.steps,
                                                  args.warmup)}))
        return
    be = hip.Backend(precision="bf16")

    def calibration_copy():
        """One device-to-device copy of exactly COPY_BYTES (the runtime's
        copy kernel reads and writes that many bytes): the reference point
        that scales the HBM byte counters of a profiling run."""
        src = be.alloc(COPY_BYTES, "copy src")
        dst = be.alloc(COPY_BYTES, "copy dst")
        be.copy(src, dst, 0, 0, COPY_BYTES)
        be.finish()
        be.release(src)
        be.release(dst)

    if args.one_window_only:
        # One 576-token window of 16 heads: the bf16 grouped launch, then
        # the exact path's launch with its key splits merged inside it.
        be32 = hip.Backend(precision="fp32")
        one = Block(hip, be, 24, seed=1, grid=24)
        one.region()
        be.finish()
        one32 = Block(hip, be32, 24, seed=1, grid=24)
        one32.region()
        be32.finish()
        ms = timed(be, one.attn, args.steps, args.warmup)
        ms32 = timed(be32, one32.attn_f32, args.steps, args.warmup)
        print(json.dumps({"kernel": "attention, one window 576 x 16 heads",
                          "bf16_ms": ms, "fp32_ms": ms32,
                          "bf16_TFLOP/s": one.flops() / ms / 1e9,
                          "fp32_TFLOP/s": one.flops() / ms32 / 1e9}))
        return
    if args.window_only:
        win = Block(hip, be, 24, seed=2)
        win.region()
        be.finish()
        calibration_copy()
        ms = timed(be, win.attn, args.steps, args.warmup)
        print(json.dumps({"kernel": "attn_bf16 windowed 9x576", "ms": ms,
                          "TFLOP/s": win.flops() / ms / 1e9}))
        return
    glob = Block(hip, be, 0, seed=3)
    glob.region()          # LN -> QKV -> pack -> attention; packs operands
    be.finish()
    if args.kernel_only or args.region_only:
        calibration_copy()
        fn = glob.attn if args.kernel_only else glob.region
        ms = timed(be, fn, args.steps, args.warmup)
        print(json.dumps({"kernel": "attn_bf16 global" if args.kernel_only
                          else "attention region global", "ms": ms,
                          "TFLOP/s": glob.flops() / ms / 1e9}))
        return

    # Host-side sections first (the GPU idles meanwhile): the decoder
    # oracle on the host cores and the checkpoint upload timings.
    mdec_cpu = None if args.no_cpu else mask_decoder_cpu()
    ckpt = checkpoint_load(hip)
    win = Block(hip, be, 24, seed=2)
    win.region()
    be.finish()
    sub_steps, sub_warm = max(5, args.steps // 5), max(2, args.warmup // 10)
    be32 = hip.Backend(precision="fp32")
    # Config 1: one 576-token window (16 heads), the shape the reference's
    # own CPU run takes, and its exact path. Built here, so that their timed
    # launches follow the windowed line's with no host work between them
    # (a 9 us kernel timed from a dropped engine clock reads 20-25 % slow).
    one = Block(hip, be, 24, seed=1, grid=24)
    one.region()
    be.finish()
    one32 = Block(hip, be32, 24, seed=1, grid=24)
    one32.region()
    be32.finish()

    # GPU sections: fp32 exact path (f32 MFMA, same shapes, its own
    # backend), decoder attention, mask decoder, text path, backbone.
    g32 = Block(hip, be32, 0, seed=3)
    g32.region()
    be32.finish()
    g32_ms = timed(be32, g32.attn_f32, max(3, args.steps // 10), sub_warm)
    w32 = Block(hip, be32, 24, seed=2)
    w32.region()
    be32.finish()
    w32_ms = timed(be32, w32.attn_f32, max(3, args.steps // 10), sub_warm)
    dec = decoder(hip, be32, sub_steps, sub_warm)
    mdec = mask_decoder(hip, max(3, sub_steps // 2), 2)
    if mdec_cpu is not None:
        mdec["cpu_oracle"] = mdec_cpu
    text = text_attention(hip, sub_steps, sub_warm)
    bb = backbone(hip, 5, 2)
    # Clock conditioning: the sections above end in host work (reading
    # profiles, freeing buffers), after which the engine clock has dropped; from there it takes 10-20 ms of sustained work to
    # come back (the global kernel runs 122 us after 5 warm-up launches
    # from idle, 110.6 us after 200). The global block's attention region,
    # replayed back to back for ~27 ms, brings it to its loaded state
    # before the W warm-up steps of the headline.
    for _ in range(COND_REGIONS):
        glob.region()
    be.finish()

    # The headline: W warm-up launches, then exactly K timed launches of the
    # global attention, right after the GPU sections above, so the engine
    # clock is at its loaded steady state rather than ramping from idle
    # within the short timed region; then the windowed batch under the same
    # protocol: COND_REGIONS replays of its own block's attention region,
    # W warm-up launches and, its launches being a sixth as long, 6 K timed
    # ones (20 launches of a 17 us kernel are too short a window).
    ms = timed(be, glob.attn, args.steps, args.warmup)
    tflops = glob.flops() / ms / 1e9
    for _ in range(COND_REGIONS):
        win.region()
    be.finish()
    wms = timed(be, win.attn, 6 * args.steps, args.warmup)
    # Config 1 right after, the engine still loaded: 6 K launches each (a
    # launch of the bf16 window is half the windowed batch's).
    one_ms = timed(be, one.attn, 6 * args.steps, args.warmup)
    one32_ms = timed(be32, one32.attn_f32, 6 * args.steps, args.warmup)
    region_ms = timed(be, glob.region, sub_steps, sub_warm)
    qkv_ms = timed(be, glob.qkv_gemm, sub_steps, sub_warm)
    w_region = timed(be, win.region, sub_steps, sub_warm)

    qkv_flops = 2.0 * 5184 * 1024 * 3072
    result = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (x ~ N(0,1), LayerNorm, Xavier-uniform QKV, "
                "axial RoPE theta 1e4; random init)",
        "config": {"workload": "global self-attention of one ViT block: 5184 "
                               "tokens (72x72), 16 heads x 64, 2D RoPE, bf16 "
                               "MFMA f32 accumulate",
                   "tokens": 5184, "heads": 16, "head_dim": 64,
                   "parallelism": "none (1 GPU)"},
        "pct_bf16_peak": round(100 * tflops / PEAK_BF16, 2),
        "clock_conditioning": "%d back-to-back replays of the global block's attention "
                              "region (LayerNorm, QKV projection, attention; ~27 ms) "
                              "before the W warm-up steps" % COND_REGIONS,
        "windowed": {"workload": "9 windows x 576 tokens, 16 heads x 64, bf16",
                     "ms": round(wms, 5), "launches_timed": 6 * args.steps,
                     "warmup_launches": args.warmup,
                     "clock_conditioning": "%d replays of the windowed block's "
                                           "attention region" % COND_REGIONS,
                     "TFLOP/s": round(win.flops() / wms / 1e9, 2),
                     "pct_bf16_peak": round(100 * win.flops() / wms / 1e9 /
                                            PEAK_BF16, 2),
                     "region_ms": round(w_region, 4)},
        "single_window": {"workload": "1 window x 576 tokens, 16 heads x 64",
                          "bf16_ms": round(one_ms, 5),
                          "bf16_TFLOP/s": round(one.flops() / one_ms / 1e9, 2),
                          "fp32_ms": round(one32_ms, 5),
                          "fp32_TFLOP/s": round(one.flops() / one32_ms / 1e9, 2),
                          "launches_timed": 6 * args.steps,
                          "warmup_launches": args.warmup},
        "global_region_ms": round(region_ms, 4),
        "qkv_gemm_bf16": {"ms": round(qkv_ms, 4),
                          "TFLOP/s": round(qkv_flops / qkv_ms / 1e9, 1)},
        "fp32_exact": {
            "global_ms": round(g32_ms, 4),
            "global_TFLOP/s": round(glob.flops() / g32_ms / 1e9, 2),
            "global_pct_f32_peak": round(100 * glob.flops() / g32_ms / 1e9 /
                                         PEAK_F32, 1),
            "windowed_ms": round(w32_ms, 4),
            "windowed_TFLOP/s": round(win.flops() / w32_ms / 1e9, 2)},
        "decoder_fp32": dec,
        "mask_decoder": mdec,
        "backbone": bb,
        "text_attention": text,
        "checkpoint": ckpt,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                     "peak": PEAK_BF16, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16, 4),
                     "traffic": round(1024 * (ATTN_FETCH_KIB * FETCH_SCALE +
                                              ATTN_WRITE_KIB * WRITE_SCALE)),
                     "traffic_algorithmic": glob.bytes(),
                     "kernel": "k_attn_bf16 (global, 5184 tokens x 16 heads)",
                     "flops_per_launch": glob.flops()},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
        result["cpu_configs"] = cpu_configs()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
