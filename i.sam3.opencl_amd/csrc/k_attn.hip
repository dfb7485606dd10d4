/* SPDX-License-Identifier: Unlicense
 *
 * Fused softmax attention on gfx950 (head width 64), replacing the
 * reference's gemm(Q K^T) -> softmax_rows -> gemm(P V) sequence
 * (sam3_model.c:1000-1013) for windowed and global ViT blocks.
 *
 * Both kernels compute S^T = K Q^T and O^T = V^T P^T rather than S and O:
 * in the 32 x 32 MFMA output layout a lane then holds one query (column
 * l % 32) and 16 of its keys, so the row max / row sum need one exchange
 * between lanes l and l ^ 32, the per-query rescale of O is a per-lane
 * scalar, and P feeds the P V product straight from registers.
 *
 * Workgroup: 256 threads = 4 waves; each wave owns 32 queries, the
 * workgroup 128 queries of one (window, head) unit (blockIdx.y). K and V
 * blocks are staged through double-buffered LDS with the next block
 * prefetched into registers while the current one is consumed. The
 * online softmax keeps (m, l) per lane: m is the running max of the
 * scaled scores, l the partial sum over the lane's keys; the halves are
 * combined once at the end.
 *
 * MFMA 32x32 lane layouts (l = lane, h = l / 32):
 *   A operand:  lane l holds A[l % 32][k-slice h]
 *   B operand:  lane l holds B[k-slice h][l % 32]
 *   D (16 f32): reg r of lane l is D[8 (r / 4) + 4 h + r % 4][l % 32]
 */
#include "k_common.h"

#include <type_traits>

/* XCDs (L2 domains) of an MI355X: workgroup i of a launch runs on XCD
 * i % NXCD. */
#define NXCD 8

/* Word 3 of a raw buffer resource (gfx9: 32-bit data format, no
 * swizzle), and the sc1 cache policy of the buffer loads and stores that
 * agent-scope atomics also carry (coherent across the XCDs' L2s). */
#define BUF_RSRC_DW3 0x00020000
#define CPOL_SC1 16

/* Key splits of one (unit, query tile) merged inside their launch, in two
 * levels: the splits form groups of SPLIT_GROUP (the last group may be
 * shorter); the last split of a group to arrive folds the group's records
 * into a group record, and the last group to finish folds the group
 * records (one group: the group's fold is the result). Every fold takes
 * its records in order, three at a time, into a running (M, L, O) as the
 * online softmax folds blocks: M the largest m so far over records that
 * saw a key (l > 0), O and L rescaled by 2^(M_old - M) and the record's o
 * and l added with weight 2^(m_r - M); a record that saw no key adds
 * nothing. Every record comes back from memory, the folding workgroup's
 * own included, so the bits do not depend on which split or group
 * arrives last; two levels spread the reading over up to nine
 * workgroups' CUs instead of one.
 *
 * Records: per tile (item) SPLIT_RECS(nsplit) of them at part + item
 * SPLIT_RECS(nsplit) 9216 floats, the nsplit split records, then the
 * group records; per record and wave nine 16-byte chunks per lane,
 * chunk-major (chunk c of lane l at byte 16 (64 c + l), so that each
 * chunk of a wave is one coalesced KiB): O^T registers 4 c .. 4 c + 3 of
 * o0 in chunks 0-3 and of o1 in 4-7 (O1), (m in log2 units, l of the whole
 * query) in chunk 8. Stored and loaded with the sc1 policy of agent-scope
 * atomics (coherent across the XCDs' L2s); a workgroup counts itself in
 * (cnt[item SPLIT_CNT + group], then cnt[item SPLIT_CNT + SPLIT_GROUP] for
 * the groups) once its stores are done (vmcnt(0), then the barrier), and
 * each last arrival resets the count it read. The loads of three records
 * are all issued before the first is used: the empty asm statements that
 * take them also order memory, so no load moves past them (left to itself
 * the scheduler waited for each load in turn).
 *
 * Returns true in the final folding workgroup's waves that store (o0, o1,
 * m, lq then hold the merged state), false elsewhere. Every wave of the
 * workgroup calls it; a wave with store false (no query of its own)
 * meets the barriers but leaves no record and folds nothing. */
template <bool O1>
__device__ __forceinline__ bool split_merge(float *__restrict__ part, unsigned *__restrict__ cnt,
                                            long item, int nsplit, int sp, bool store,
                                            f32x16 &o0, f32x16 &o1, float &m, float &lq)
{
    __shared__ unsigned arrived;
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    const int ngroups = (nsplit + SPLIT_GROUP - 1) / SPLIT_GROUP, nrec = nsplit + ngroups;
    const int g = sp / SPLIT_GROUP, g0 = g * SPLIT_GROUP;
    const int gn = nsplit - g0 < SPLIT_GROUP ? nsplit - g0 : SPLIT_GROUP;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        part + item * nrec * 9216, (short)0, nrec * 9216 * 4, BUF_RSRC_DW3);
    unsigned *const cg = cnt + item * SPLIT_CNT;
    auto off = [&](int r, int c) { return ((r * 4 + w) * 9 + c) * 1024 + 16 * l; };
    auto put = [&](int r) {
        for (int c = 0; c < 4; c++) {
            const f32x4 x0 = {o0[4 * c], o0[4 * c + 1], o0[4 * c + 2], o0[4 * c + 3]};

            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x0), rs, off(r, c),
                                                   0, CPOL_SC1);
            if (O1) {
                const f32x4 x1 = {o1[4 * c], o1[4 * c + 1], o1[4 * c + 2], o1[4 * c + 3]};

                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x1), rs,
                                                       off(r, 4 + c), 0, CPOL_SC1);
            }
        }
        const f32x4 ml = {m, lq, 0.0f, 0.0f};

        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ml), rs, off(r, 8), 0,
                                               CPOL_SC1);
    };
    /* Counts the workgroup in at *c after its stores; true in the last of
     * n arrivals, which resets the count. */
    auto count_in = [&](unsigned *c, int n) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (t == 0)
            arrived = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (arrived != (unsigned)(n - 1))
            return false;
        if (t == 0)
            __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    };
    /* Folds records r0 .. r0 + n - 1 into (o0, o1, m, lq). */
    auto fold = [&](int r0, int n) {
        float M = -INFINITY, L = 0.0f;
        f32x16 a0, a1;

        for (int r = 0; r < 16; r++) {
            a0[r] = 0.0f;
            a1[r] = 0.0f;
        }
        for (int s0 = 0; s0 < n; s0 += 3) {
            u32x4 ch[3][9];

            for (int j = 0; j < 3; j++) {
                const int r = r0 + (s0 + j < n ? s0 + j : s0);

                for (int c = 0; c < 9; c++)
                    ch[j][c] = O1 || c < 4 || c == 8
                                   ? __builtin_amdgcn_raw_buffer_load_b128(rs, off(r, c), 0,
                                                                           CPOL_SC1)
                                   : u32x4{0u, 0u, 0u, 0u};
            }
            for (int j = 0; j < 3; j++) {
                asm volatile("" : "+v"(ch[j][0]), "+v"(ch[j][1]), "+v"(ch[j][2]),
                             "+v"(ch[j][3]), "+v"(ch[j][4]), "+v"(ch[j][5]), "+v"(ch[j][6]),
                             "+v"(ch[j][7]), "+v"(ch[j][8])::"memory");
                const f32x4 ml = __builtin_bit_cast(f32x4, ch[j][8]);
                const bool take = ml[1] > 0.0f && s0 + j < n;
                const float Mn = take ? fmaxf(M, ml[0]) : M;
                const float c = take ? __builtin_amdgcn_exp2f(M - Mn) : 1.0f;
                const float wt = take ? __builtin_amdgcn_exp2f(ml[0] - Mn) : 0.0f;

                for (int q = 0; q < 4; q++) {
                    const f32x4 v0 = __builtin_bit_cast(f32x4, ch[j][q]);
                    const f32x4 v1 = __builtin_bit_cast(f32x4, ch[j][4 + q]);

                    for (int e = 0; e < 4; e++) {
                        a0[4 * q + e] = fmaf(v0[e], wt, a0[4 * q + e] * c);
                        if (O1)
                            a1[4 * q + e] = fmaf(v1[e], wt, a1[4 * q + e] * c);
                    }
                }
                L = fmaf(ml[1], wt, L * c);
                M = Mn;
            }
        }
        o0 = a0;
        o1 = a1;
        m = M;
        lq = L;
    };

    /* Level 0: this split's record, its group's count and fold; level 1
     * (more than one group): the group's record, the groups' count and
     * fold. One loop, so that the store and the fold are emitted once. */
    int rec = sp, r0 = g0, n = gn;
    unsigned *c = cg + g;

    for (int lev = 0;; lev++) {
        if (store)
            put(rec);
        if (!count_in(c, n))
            return false;
        if (store)
            fold(r0, n);
        if (lev == 1 || ngroups == 1)
            return store;
        rec = nsplit + g;
        r0 = nsplit;
        n = ngroups;
        c = cg + SPLIT_GROUP;
    }
}

/* Scores may run this far (log2 units) above or below the reference
 * point m before it must move: exp2 of them stays far inside the float
 * and bf16 ranges, and the accumulated O and l with it (5184 keys x 2^64
 * x |v|). */
#define SAFE_SPAN 64.0f

/* Box relative position bias of softmax_ext (sam3_kernels.cl:885-921)
 * added to registers r0 .. r0 + RUN - 1 of s, the scores of keys j0 ..
 * j0 + RUN - 1 of one query, j0 = y W + x (x < W, both multiples of RUN;
 * W a multiple of RUN, so the run lies in one grid row and is either all
 * below Nk or all past it, where nothing is added: those keys are
 * masked): dy[y] + dx[x + e] from the query's row of the bias rows (H =
 * Nk / W values of dy, then W >= 64 of dx, H a multiple of 4:
 * launch_box_rows), one dy value and RUN / 4 16-byte runs of dx. The
 * caller finds (y, x) from the block's first key without a division per
 * run (block_yx). Other grids take the bias as a table (launch_box_bias). */
template <int RUN>
__device__ __forceinline__ void box_add(const float *__restrict__ row, int H, int Nk, int j0,
                                        int y, int x, f32x16 &s, int r0)
{
    if (j0 >= Nk)
        return;
    const float yv = row[y];

    for (int q = 0; q < RUN / 4; q++) {
        const f32x4 xv = *(const f32x4 *)(row + H + x + 4 * q);

        for (int e = 0; e < 4; e++)
            s[r0 + 4 * q + e] += yv + xv[e];
    }
}

/* (y, x) of key jb + off for a block's first key jb = yb W + xb, for
 * off < 64 <= W (one wrap at most). */
__device__ __forceinline__ void block_yx(int yb, int xb, int W, int off, int &y, int &x)
{
    y = yb;
    x = xb + off;
    if (x >= W) {
        x -= W;
        y++;
    }
}

/* ------------------------------------------------------------ fp32 path */

/* fp32 operands in the reference row layout (Q/K/V/O opnds of
 * sam3_model.c:1004-1011, or the Q, K, V, O rows of the text path's
 * attend, sam3_text.c:305-343), v_mfma_f32_32x32x2_f32, 32-key blocks:
 * the exact path. N queries over Nk keys per unit, head width HD (64, or
 * 32 for the text path's heads). RoPE (HD 64) is applied on the loads,
 * the scale to the scores. The contraction index of Q K^T is ordered
 * d = step + (HD / 2) h, so a lane's Q registers are one contiguous half
 * row and RoPE pairs stay in one lane.
 *
 * EXT adds softmax_ext's terms (sam3_kernels.cl:885-921) the way it adds
 * them: the causal mask (key j > query i: -inf), or the box bias dy + dx
 * from the bias rows of launch_box_rows (d.bW = W), or from an additive
 * table [unit][N][Nk padded to 64] of the sums (k_box_bias with scale 1,
 * d.bW = 0), added to the scaled score as softmax_ext adds it.
 *
 * With nsplit > 1 (the SPLIT instance) the workgroup takes key blocks
 * [kb0, kb1) of split sp and the tile's splits merge inside the launch
 * (split_merge; `part` holds nb, 128-query tiles, SPLIT_RECS(nsplit)
 * records of 9216 floats, cnt SPLIT_CNT counts per (unit, tile)): the
 * final folding workgroup stores O. A query none of whose keys a split
 * sees (causal) has l = 0 there and drops out of the merge. */
template <int HD, bool EXT, bool SPLIT>
__global__ __launch_bounds__(256) void k_attn_f32(attn_desc d, float *__restrict__ part,
                                                  unsigned *__restrict__ cnt, int nsplit)
{
    __shared__ float Kt[2][HD][33]; /* K^T block: [d][key] */
    __shared__ float Vs[2][32][HD + 8]; /* V block:   [key][d] */
    constexpr int HH = HD / 2;          /* channels per lane half */
    constexpr int LPR = HD / 8;         /* loader threads per key row */
    const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5,
              l32 = l & 31;
    const int N = d.N, Nk = d.Nk;
    /* (unit, tile, split) triples in that order, in NXCD contiguous
     * ranges, one per XCD: the splits of a tile and the tiles of a unit
     * share one L2 (their Q rows, K and V blocks). */
    const int ntiles = (N + 127) / 128;
    const long total = (long)d.nb * ntiles * nsplit, per = (total + NXCD - 1) / NXCD;
    const long pos = (long)(blockIdx.x % NXCD) * per + blockIdx.x / NXCD;

    if (pos >= total)
        return;
    const long item = pos / nsplit, unit = item / ntiles;
    const int sp = (int)(pos - item * nsplit), tile = (int)(item - unit * ntiles);
    const long b0 = unit / d.nb1, b1 = unit % d.nb1;
    const float *Qb = (const float *)d.Q + d.qoff + b0 * d.sq0 + b1 * d.sq1;
    const float *Kb = (const float *)d.K + d.koff + b0 * d.sk0 + b1 * d.sk1;
    const float *Vb = (const float *)d.V + d.voff + b0 * d.sv0 + b1 * d.sv1;
    const float2 *cs = (const float2 *)d.rope;
    const int qi = tile * 128 + w * 32 + l32;
    /* A wave whose 32 queries all lie past N (the tail tile's): its
     * scores are computed and dropped (a branch around the block's
     * arithmetic would keep the staging stores from overlapping the P V
     * product), but it leaves no split record. */
    const bool idle = tile * 128 + __builtin_amdgcn_readfirstlane(w) * 32 >= N;
    const int nblk = (Nk + 31) / 32;
    const int kb0 = (int)((long)sp * nblk / nsplit), kb1 = (int)((long)(sp + 1) * nblk / nsplit);
    /* This lane's row of the bias table, if any (queries past N read the
     * last row, never stored). */
    const int bH = d.bW > 0 ? Nk / d.bW : 0;
    const float *brow = EXT && d.bias
                            ? d.bias + ((long)unit * N + (qi < N ? qi : N - 1)) *
                                           (d.bW > 0 ? bH + d.bW : (Nk + 63) / 64 * 64)
                            : nullptr;
    /* Loader role: key row kr of a block, 8 channels from dc; with HD 32
     * the upper half of the threads loads nothing. */
    const int kr = t / LPR, dc = (t % LPR) * 8;
    const bool loader = t < 32 * LPR;
    float qreg[HH], kpre[8], vpre[8];
    f32x16 o0, o1;
    float m_run = 0.0f, l_run = 0.0f;
    const float sc2 = d.scale * LOG2E_F;

    /* Q: lane holds channels HH h .. HH h + HH - 1 of query qi, rotated
     * and scaled. */
    for (int i = 0; i < HH; i++)
        qreg[i] = 0.0f;
    if (qi < N) {
        const float *qr = Qb + (long)qi * d.ldq + HH * h;

        for (int i = 0; i < HH; i++)
            qreg[i] = qr[i];
        if (HD == 64 && cs) {
            const float2 *rot = cs + (long)(qi % d.npos) * 32 + 16 * h;

            for (int j = 0; j < HH / 2; j++) {
                const float a = qreg[2 * j], b = qreg[2 * j + 1];
                const float2 r = rot[j];

                qreg[2 * j] = fmaf(a, r.x, -(b * r.y));
                qreg[2 * j + 1] = fmaf(a, r.y, b * r.x);
            }
        }
    }
    for (int r = 0; r < 16; r++) {
        o0[r] = 0.0f;
        o1[r] = 0.0f;
    }

    /* Global -> registers for block kb (RoPE on K), registers -> LDS. */
    auto fetch = [&](int kb) {
        const int key = kb * 32 + kr;

        if (loader && key < Nk) {
            const float *kp = Kb + (long)key * d.ldk + dc;
            const float *vp = Vb + (long)key * d.ldv + dc;

            for (int e = 0; e < 8; e++) {
                kpre[e] = kp[e];
                vpre[e] = vp[e];
            }
            if (HD == 64 && cs) {
                const float2 *rot = cs + (long)(key % d.npos) * 32 + dc / 2;

                for (int j = 0; j < 4; j++) {
                    const float a = kpre[2 * j], b = kpre[2 * j + 1];
                    const float2 r = rot[j];

                    kpre[2 * j] = fmaf(a, r.x, -(b * r.y));
                    kpre[2 * j + 1] = fmaf(a, r.y, b * r.x);
                }
            }
        }
        else
            for (int e = 0; e < 8; e++) {
                kpre[e] = 0.0f;
                vpre[e] = 0.0f;
            }
    };
    auto stage = [&](int buf) {
        if (loader)
            for (int e = 0; e < 8; e++) {
                Kt[buf][dc + e][kr] = kpre[e];
                Vs[buf][kr][dc + e] = vpre[e];
            }
    };

    /* S^T = K Q^T of the block in buffer buf (unscaled). */
    auto qk = [&](int buf) {
        f32x16 s;

        for (int r = 0; r < 16; r++)
            s[r] = 0.0f;
#pragma unroll
        for (int st = 0; st < HH; st++)
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(Kt[buf][st + HH * h][l32], qreg[st], s, 0,
                                                     0, 0);
        return s;
    };
    /* Scores in log2 units relative to the lane's reference point m
     * (m_run, log2 units, the same in lanes l and l ^ 32): t = s scale
     * log2(e) - m as one rounding, keys past Nk (last block), the causal
     * mask or the bias (added to the scaled score, natural units, as
     * softmax_ext adds it) applied; then P = exp2(t), O^T += V^T P^T from
     * buffer buf. Register r holds key kb 32 + 8 (r / 4) + 4 h + r % 4.
     * m is the first block's max, then moves only when a score leaves
     * [m - SAFE_SPAN, m + SAFE_SPAN]: up (O and l shrink) when the block
     * max passes m + SAFE_SPAN, down while the query has no weight yet
     * and its block max lies below m - SAFE_SPAN. After the first block a
     * wave takes the exact max (its cross-lane exchange, the rescale of O
     * and l) only for blocks whose in-lane maxima it cannot clear; O / l
     * does not depend on m. */
    auto soft_pv = [&](f32x16 s, int kb, int buf) {
        float rs = 0.0f, mx = -INFINITY;

        if (EXT && brow) {
            for (int r = 0; r < 16; r++)
                s[r] *= d.scale;
            if (d.bW > 0) {
                const int yb = kb * 32 / d.bW, xb = kb * 32 - yb * d.bW;

                for (int g = 0; g < 4; g++) {
                    int y, x;

                    block_yx(yb, xb, d.bW, 8 * g + 4 * h, y, x);
                    box_add<4>(brow, bH, Nk, kb * 32 + 8 * g + 4 * h, y, x, s, 4 * g);
                }
            }
            else
                for (int g = 0; g < 4; g++) {
                    const f32x4 bv = *(const f32x4 *)(brow + kb * 32 + 8 * g + 4 * h);

                    for (int e = 0; e < 4; e++)
                        s[4 * g + e] += bv[e];
                }
            for (int r = 0; r < 16; r++)
                s[r] = fmaf(s[r], LOG2E_F, -m_run);
        }
        else
            for (int r = 0; r < 16; r++)
                s[r] = fmaf(s[r], sc2, -m_run);
        if (kb * 32 + 32 > Nk)
            for (int r = 0; r < 16; r++) {
                const int key = kb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);

                s[r] = key < Nk ? s[r] : -INFINITY;
            }
        if (EXT && d.causal)
            for (int r = 0; r < 16; r++) {
                const int key = kb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);

                if (key > qi)
                    s[r] = -INFINITY;
            }
        for (int r = 0; r < 16; r++)
            mx = fmaxf(mx, s[r]);
        if (kb == kb0 || __ballot(mx > SAFE_SPAN || (l_run == 0.0f && mx < -SAFE_SPAN &&
                                                    mx != -INFINITY)) != 0) {
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const bool empty = l_run + __shfl_xor(l_run, 32, 64) == 0.0f;
            /* The first block sets m to its max outright, as the reference's
             * softmax does (that key's weight is then exactly 1: a query
             * that sees one key gets its value row unchanged). */
            const float mv = (kb == kb0 || mx > SAFE_SPAN || (empty && mx < -SAFE_SPAN)) &&
                                     mx != -INFINITY
                                 ? mx
                                 : 0.0f;

            if (kb != kb0) {
                /* Moving down, the query has no weight to rescale. */
                const float corr = __builtin_amdgcn_exp2f(-fmaxf(mv, 0.0f));

                l_run *= corr;
                for (int r = 0; r < 16; r++) {
                    o0[r] *= corr;
                    if (HD == 64)
                        o1[r] *= corr;
                }
            }
            for (int r = 0; r < 16; r++)
                s[r] -= mv;
            m_run += mv;
        }
        for (int r = 0; r < 16; r++) {
            s[r] = __builtin_amdgcn_exp2f(s[r]);
            rs += s[r];
        }
        l_run += rs;
        /* The exponentials issued before the P V MFMAs: left to the
         * scheduler, which weighs the code after the key loop too, each
         * MFMA could follow the exponential it reads and wait for it
         * (3 % on one 576-token window). */
        __builtin_amdgcn_sched_barrier(0);
        /* O^T += V^T P^T: step st contracts key 8 (st / 4) + 4 h + st % 4,
         * the key of this lane's score register st. */
#pragma unroll
        for (int st = 0; st < 16; st++) {
            const int key = 8 * (st >> 2) + 4 * h + (st & 3);

            o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[buf][key][l32], s[st], o0, 0, 0, 0);
            if (HD == 64)
                o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[buf][key][32 + l32], s[st], o1, 0,
                                                          0, 0);
        }
    };

    fetch(kb0);
    stage(0);
    __syncthreads();
    int lvl = -1;

    /* Two buffers: block kb + 1 is fetched while block kb is used and
     * staged after it. */
    for (int kb = kb0; kb < kb1; kb++) {
        const int buf = (kb - kb0) & 1;

        prio_by_progress(kb - kb0, kb1 - kb0, lvl);
        if (kb + 1 < kb1)
            fetch(kb + 1);
        soft_pv(qk(buf), kb, buf);
        if (kb + 1 < kb1)
            stage(buf ^ 1);
        __syncthreads();
    }
    __builtin_amdgcn_s_setprio(0);

    l_run += __shfl_xor(l_run, 32, 64);
    if constexpr (SPLIT)
        if (!split_merge<HD == 64>(part, cnt, item, nsplit, sp, !idle, o0, o1, m_run, l_run))
            return;
    if (qi >= N)
        return;
    {
        const float inv = 1.0f / l_run;
        const long orow = d.ooff + b0 * d.so0 + b1 * d.so1 + (long)qi * d.ldo;

        if (d.odt == DT_F32 && ((orow & 3) | ((uintptr_t)d.O & 15)) == 0) {
            /* Registers 4 g .. 4 g + 3 are columns 8 g + 4 h .. + 3 of the
             * lane's query row: one 16-byte store each. */
            float *op = (float *)d.O + orow + 4 * h;

            for (int g = 0; g < 4; g++) {
                const f32x4 x0 = {o0[4 * g] * inv, o0[4 * g + 1] * inv, o0[4 * g + 2] * inv,
                                  o0[4 * g + 3] * inv};

                *(f32x4 *)(op + 8 * g) = x0;
                if (HD == 64) {
                    const f32x4 x1 = {o1[4 * g] * inv, o1[4 * g + 1] * inv,
                                      o1[4 * g + 2] * inv, o1[4 * g + 3] * inv};

                    *(f32x4 *)(op + 32 + 8 * g) = x1;
                }
            }
            return;
        }
        for (int r = 0; r < 16; r++) {
            const int dd = 8 * (r >> 2) + 4 * h + (r & 3);

            if (d.odt == DT_F32) {
                ((float *)d.O)[orow + dd] = o0[r] * inv;
                if (HD == 64)
                    ((float *)d.O)[orow + 32 + dd] = o1[r] * inv;
            }
            else {
                ((uint16_t *)d.O)[orow + dd] = f2bf(o0[r] * inv);
                if (HD == 64)
                    ((uint16_t *)d.O)[orow + 32 + dd] = f2bf(o1[r] * inv);
            }
        }
    }
}

/* ------------------------------------------------------------ packing */

/* fp32 reference-layout Q/K/V -> packed bf16 of the fast path, 64 rows
 * of one unit per workgroup: q16/k16 [unit][Np][64] with RoPE applied
 * (q also scaled by scale * log2 e, so Q K^T comes out in log2 units for
 * exp2), vt16 [unit][64][Np] transposed through LDS; rows past N are
 * zero. */
__global__ __launch_bounds__(256) void k_qkv_pack(attn_desc d,
                                                  uint16_t *__restrict__ q16,
                                                  uint16_t *__restrict__ k16,
                                                  uint16_t *__restrict__ vt16,
                                                  float *__restrict__ knorm,
                                                  int Npq, int Npk)
{
    __shared__ uint16_t Vl[64][66];
    __shared__ float kred[4];
    const int t = threadIdx.x, row = t >> 2, ds = (t & 3) * 16;
    const int unit = blockIdx.y, i = blockIdx.x * 64 + row;
    const long b0 = unit / d.nb1, b1 = unit % d.nb1;
    const float2 *cs = (const float2 *)d.rope;
    /* Row blocks past one side's padded length write nothing of it. */
    const bool qblk = blockIdx.x * 64 < Npq, kblk = blockIdx.x * 64 < Npk;
    const bool qrow = i < d.N && ds < d.hd, krow = i < d.Nk && ds < d.hd;
    float q[16], k[16], v[16];

    for (int e = 0; e < 16; e++) {
        q[e] = 0.0f;
        k[e] = 0.0f;
        v[e] = 0.0f;
    }
    if (qrow) {
        const float *qr = (const float *)d.Q + d.qoff + b0 * d.sq0 +
                          b1 * d.sq1 + (long)i * d.ldq + ds;

        for (int e = 0; e < 16; e++)
            q[e] = qr[e];
    }
    if (krow) {
        const float *kr = (const float *)d.K + d.koff + b0 * d.sk0 +
                          b1 * d.sk1 + (long)i * d.ldk + ds;
        const float *vr = (const float *)d.V + d.voff + b0 * d.sv0 +
                          b1 * d.sv1 + (long)i * d.ldv + ds;

        for (int e = 0; e < 16; e++) {
            k[e] = kr[e];
            v[e] = vr[e];
        }
    }
    if (cs && (qrow || krow)) {
        const float2 *rot = cs + (long)(i % d.npos) * 32 + ds / 2;

        for (int j = 0; j < 8; j++) {
            const float2 r = rot[j];
            float a = q[2 * j], b = q[2 * j + 1];

            q[2 * j] = fmaf(a, r.x, -(b * r.y));
            q[2 * j + 1] = fmaf(a, r.y, b * r.x);
            a = k[2 * j];
            b = k[2 * j + 1];
            k[2 * j] = fmaf(a, r.x, -(b * r.y));
            k[2 * j + 1] = fmaf(a, r.y, b * r.x);
        }
    }
    for (int e = 0; e < 16; e++)
        q[e] *= d.scale * LOG2E_F;
    {
        u32x4 a, b;

        if (qblk) {
            const long o = ((long)unit * Npq + i) * 64 + ds;

            for (int e = 0; e < 4; e++) {
                a[e] = pack_bf16x2(q[2 * e], q[2 * e + 1]);
                b[e] = pack_bf16x2(q[8 + 2 * e], q[8 + 2 * e + 1]);
            }
            *(u32x4 *)(q16 + o) = a;
            *(u32x4 *)(q16 + o + 8) = b;
        }
        if (kblk) {
            const long o = ((long)unit * Npk + i) * 64 + ds;

            for (int e = 0; e < 4; e++) {
                a[e] = pack_bf16x2(k[2 * e], k[2 * e + 1]);
                b[e] = pack_bf16x2(k[8 + 2 * e], k[8 + 2 * e + 1]);
            }
            *(u32x4 *)(k16 + o) = a;
            *(u32x4 *)(k16 + o + 8) = b;
        }
    }
    {
        /* Largest |k| of this 64-key block, over the bf16 values the
         * attention multiplies: squares summed over the row's 4 threads,
         * max over the 4 waves' 16 rows each. */
        float ss = 0.0f, mx;

        for (int e = 0; e < 16; e++) {
            const float kv = bf2f(f2bf(k[e]));

            ss = fmaf(kv, kv, ss);
        }
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        mx = wave_max(ss);
        if ((t & 63) == 0)
            kred[t >> 6] = mx;
    }
    for (int e = 0; e < 16; e++)
        Vl[ds + e][row] = f2bf(v[e]);
    __syncthreads();
    if (kblk) {
        /* Thread t writes channel t / 4, keys 16 (t % 4) .. +15. */
        const int dd = t >> 2, k0 = (t & 3) * 16;
        uint16_t *dst = vt16 + ((long)unit * 64 + dd) * Npk + blockIdx.x * 64 + k0;

        for (int e = 0; e < 16; e++)
            dst[e] = Vl[dd][k0 + e];
        if (t == 0) {
            const float m2 = fmaxf(fmaxf(kred[0], kred[1]), fmaxf(kred[2], kred[3]));

            /* Rounded up by 2^-10 relative: covers the square root's and
             * the sum's roundings. */
            knorm[(long)unit * (Npk / 64) + blockIdx.x] = sqrtf(m2) * (1.0f + 0x1p-10f);
        }
    }
}

extern "C" int launch_qkv_pack(const attn_desc *d, void *q16, void *k16,
                               void *vt16, float *knorm, void *stream)
{
    const int Npq = (d->N + 63) / 64 * 64, Npk = (d->Nk + 63) / 64 * 64;
    const int Np = Npq > Npk ? Npq : Npk;

    if (d->nb > 65535 || d->Nk < 1)
        return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(k_qkv_pack, dim3(Np / 64, d->nb), dim3(256), 0,
                       (hipStream_t)stream, *d, (uint16_t *)q16,
                       (uint16_t *)k16, (uint16_t *)vt16, knorm, Npq, Npk);
    return hipGetLastError();
}

/* Bias rows of the fused attention kernels from the box relative position
 * bias of softmax_ext (sam3_kernels.cl:904-906): out[h][i] = unit_scale
 * dy[(i H + y) nh + h] for y < H, then unit_scale dx[(i W + x) nh + h] for
 * x < W (H = Nk / W), one row of H + W floats per (head, query); the
 * kernels add dy[j / W] + dx[j % W] to the score of key j (box_add)
 * instead of reading an [Nq][Nk] table per head. unit_scale 1 for the
 * exact path (the sum dy + dx softmax_ext makes), log2(e) for the bf16
 * kernel's exp2 domain. One thread per element. */
__global__ __launch_bounds__(256) void k_box_rows(float *__restrict__ out,
                                                  const float *__restrict__ dy,
                                                  const float *__restrict__ dx, int Nq,
                                                  int H, int W, int nh, long n,
                                                  float unit_scale)
{
    const long e = (long)blockIdx.x * 256 + threadIdx.x;

    if (e >= n)
        return;
    const int R = H + W, t = (int)(e % R);
    const long r = e / R;
    const int h = (int)(r / Nq), i = (int)(r - (long)h * Nq);

    out[e] = unit_scale *
             (t < H ? dy[((long)i * H + t) * nh + h] : dx[((long)i * W + (t - H)) * nh + h]);
}

extern "C" int launch_box_rows(float *out, const float *dy, const float *dx, int heads,
                               int Nq, int Nk, int W, int nh, float unit_scale,
                               void *stream)
{
    long n;

    if (heads < 1 || Nq < 1 || W < 1 || Nk % W || nh < heads)
        return hipErrorInvalidValue;
    n = (long)heads * Nq * (Nk / W + W);
    if ((n + 255) / 256 > 0x7fffffffL)
        return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(k_box_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, out, dy, dx, Nq, Nk / W, W, nh, n, unit_scale);
    return hipGetLastError();
}

/* Additive bias table of the fused attention kernels,
 * out[unit][i][j] = unit_scale (dy[(i H + j / W) nh + h] + dx[(i W + j % W)
 * nh + h]) for keys j < Nk and -inf for the padding up to Npk (unit = head
 * h, H = Nk / W): the box relative position bias of softmax_ext
 * (sam3_kernels.cl:904-906) for every (head, query, key), with unit_scale
 * log2(e) for the bf16 kernel's exp2 domain and 1 for the exact path (the
 * sum dy + dx then has softmax_ext's own rounding). */
__global__ __launch_bounds__(256) void k_box_bias(float *__restrict__ out,
                                                  const float *__restrict__ dy,
                                                  const float *__restrict__ dx,
                                                  int heads, int Nq, int Nk, int Npk,
                                                  int W, int nh, float unit_scale)
{
    /* Workgroup: one (head, query) row; its H dy and W dx values go to
     * LDS once, then the row is written as 16-byte runs of four keys. */
    extern __shared__ float sxy[];
    const int r = blockIdx.x, h = r / Nq, i = r - h * Nq, H = Nk / W;
    float *sy = sxy, *sx = sxy + H;
    float *orow = out + (long)r * Npk;

    for (int t = threadIdx.x; t < H; t += 256)
        sy[t] = dy[((long)i * H + t) * nh + h];
    for (int t = threadIdx.x; t < W; t += 256)
        sx[t] = dx[((long)i * W + t) * nh + h];
    __syncthreads();
    for (int j0 = 4 * threadIdx.x; j0 < Npk; j0 += 1024) {
        f32x4 v;

        for (int k = 0; k < 4; k++) {
            const unsigned j = j0 + k, y = j / (unsigned)W;

            v[k] = j < (unsigned)Nk ? (sy[y] + sx[j - y * W]) * unit_scale : -INFINITY;
        }
        *(f32x4 *)(orow + j0) = v;
    }
}

extern "C" int launch_box_bias(float *out, const float *dy, const float *dx,
                               int heads, int Nq, int Nk, int W, int nh,
                               float unit_scale, void *stream)
{
    const int Npk = (Nk + 63) / 64 * 64;
    const long rows = (long)heads * Nq;
    const size_t lds = ((size_t)Nk / W + W) * sizeof(float);

    if (rows == 0)
        return hipSuccess;
    if (rows > 0x7fffffffL || W < 1 || lds > 65536)
        return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(k_box_bias, dim3((unsigned)rows), dim3(256), lds,
                       (hipStream_t)stream, out, dy, dx, heads, Nq, Nk, Npk, W, nh,
                       unit_scale);
    return hipGetLastError();
}

/* ------------------------------------------------------------ bf16 path */

/* Row of the K block feeding A-operand row i: bits 2 and 3 of i swapped.
 * The S^T register r of lane half h then holds key
 * 32 c + 16 (r / 8) + 8 h + r % 8, so registers 8a .. 8a + 7 are eight
 * consecutive keys: the B operand of the P V product for keys
 * 16 (2c + a) + 8 h .. +7 without any data movement. */
__device__ __forceinline__ int kperm(int i)
{
    return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}

/* Max of 16 scores. The operands are MFMA results (or sums with a -inf
 * mask), which the compiler knows are canonical, so this becomes eight
 * v_max3_f32 without NaN-quieting canonicalisation. */
__device__ __forceinline__ float max16(const f32x16 &s, float m)
{
    for (int r = 0; r < 16; r++)
        m = __builtin_fmaxf(m, s[r]);
    return m;
}

/* Sum of the 32 weights of a block (pairwise, f32 adds). The row sums of
 * P are taken from the f32 exponentials with VALU adds rather than with
 * v_dot2_f32_bf16 on the bf16 weights: on gfx950 that dot product waits
 * for the MFMA pipe, so it stalls behind every matrix product in flight
 * on the SIMD, while plain adds issue beside them. */
__device__ __forceinline__ float sum32(const f32x16 &a, const f32x16 &b)
{
    float t[8];

    for (int i = 0; i < 8; i++)
        t[i] = (a[2 * i] + a[2 * i + 1]) + (b[2 * i] + b[2 * i + 1]);
    return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
}

/* LDS rows of K [key][d] and V^T [d][key] blocks are 64 bf16 (128 B, no
 * padding); the 16-byte chunk c of row r is stored at chunk
 * c ^ ((r >> 1) & 7). A 16-lane group of 16-byte reads then touches 16
 * distinct bank groups whenever it reads one logical chunk of 16
 * different rows (MFMA operand reads) or 8 chunks of two adjacent rows
 * (staging writes). */
__device__ __forceinline__ int swz(int row, int chunk)
{
    return 8 * (chunk ^ ((row >> 1) & 7));
}

/* Online-softmax state of one wave: 32 queries (one per lane pair l,
 * l ^ 32), O^T accumulators for d 0..31 and 32..63. */
struct SoftState {
    f32x16 o0, o1;
    float m, l;
};

/* Asynchronous 16-byte global -> LDS copy (global_load_lds_dwordx4):
 * lane i of the wave writes lds_base + 16 i (lds_base wave-uniform, via
 * M0). Issued as inline assembly so that the compiler does not treat the
 * copy as a store that later LDS reads of the other slot must wait for:
 * the kernel waits for it itself (s_waitcnt vmcnt(0)) before the barrier
 * that hands the slot to the readers. */
__device__ __forceinline__ void g2lds16(const void *g, void *lds_base)
{
    /* The low 32 bits of a flat LDS address are the LDS offset. */
    const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_base);

    asm volatile("s_mov_b32 m0, %0\n\t"
                 "global_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds), "v"(g)
                 : "memory", "m0");
}

/* The same copy with a wave-uniform 64-bit base in SGPRs and a 32-bit
 * per-lane byte offset (the saddr form): no per-lane address arithmetic
 * when only the base moves from block to block. `lds` must be
 * wave-uniform. */
__device__ __forceinline__ void g2lds16_s(const void *base, unsigned voff, unsigned lds)
{
    asm volatile("s_mov_b32 m0, %0\n\t"
                 "global_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(base)
                 : "memory", "m0");
}

/* Balanced launch of k_attn_bf16 when the tiles fill between two and
 * three workgroups per CU (the global ViT block: 82 tiles per XCD on 32
 * CUs): on each XCD, dp workgroups take one whole tile each and the
 * remaining tiles' (tile, key block) pairs are shared evenly by G more
 * workgroups (stream-K), so every CU gets about the same number of key
 * blocks instead of some three tiles and others two. rec holds 2 records
 * of 4 waves x 34 x 64 floats per stream-K workgroup (8 G of them) for
 * the pieces of cut tiles, cnt one arrival counter per tile (zero before
 * the first launch; the last piece of each tile zeroes it again). G = 0
 * turns it off. */
struct sk_desc {
    float *rec;
    unsigned *cnt;
    int G, dp;
};

/* Packed bf16 operands (k_qkv_pack layout), v_mfma_f32_32x32x16_bf16 with
 * f32 accumulation, 64-key blocks.
 *
 * Small per-wave state keeps three waves on every SIMD, so the Q K^T /
 * P V MFMAs of some waves overlap the softmax VALU work of others. K /
 * V^T blocks move HBM -> LDS with asynchronous global_load_lds (no
 * staging registers) into two swizzled slots; the next block's copy is
 * issued right after the barrier that retires the slot it overwrites, so
 * one barrier per block suffices.
 *
 * The softmax reference point m (P = exp2(s - m), O and l scaled alike,
 * so O / l does not depend on it) starts at 0 and only moves when a
 * score could leave [m - SAFE_SPAN, m + SAFE_SPAN]. |q . k| <= |q| |k|,
 * and the packing kernel records each block's largest |k|, so a wave
 * first checks the bound |q| max|k| - m <= SAFE_SPAN for all its lanes
 * (three VALU operations); only blocks it cannot clear take the exact
 * block max with its cross-lane exchange. Each query then moves its own
 * m: up to a block max above m + SAFE_SPAN (O and l shrink), or, while
 * it has no weight yet, down to a block max below m - SAFE_SPAN. Hence
 * every query's largest score so far stays within SAFE_SPAN of its m:
 * no weight exceeds 2^SAFE_SPAN and the largest is >= 2^-SAFE_SPAN, at
 * any score magnitude. While every m of the wave is 0 the scores feed
 * exp2 directly. */
/* Key blocks [kb0, kb1) of query tile `tile` of unit `unit`: the body
 * of k_attn_bf16 (a function rather than a lambda: wrapping it in a
 * lambda costs the bias variant its register budget). `d` is the
 * descriptor or, in stream-K mode, an opaque alias of it. With SPL the
 * key blocks are split sp of nsplit, merged inside the launch
 * (split_merge, counting on sk.cnt). */
template <bool EXT, bool H32, bool SK, bool SPL, class Desc>
__device__ __forceinline__ void attn_tile(const Desc &d, const uint16_t *__restrict__ q16,
                                          const uint16_t *__restrict__ k16,
                                          const uint16_t *__restrict__ vt16,
                                          const float *__restrict__ knorm,
                                          float *__restrict__ part, int nsplit, int sp,
                                          const sk_desc &sk, unsigned rank, long unit,
                                          int tile, int kb0, int kb1, int pdone, int ptotal,
                                          int rbase, int R)
{
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][64][64];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[2][64][64];
    __shared__ unsigned arrived;
    const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5,
              l32 = l & 31;
    /* N queries and Nk keys per unit, each padded to a multiple of 64. */
    const int N = d.N, Nk = d.Nk, Np = (N + 63) / 64 * 64,
              Npk = (Nk + 63) / 64 * 64, nblk = Npk / 64;
    const int ntiles = (N + 127) / 128;
    const int krow = kperm(l32);
    const f32x16 zero16 = {};
    const int wu = __builtin_amdgcn_readfirstlane(w);
    unsigned koff[2], voff[2];
    for (int j = 0; j < 2; j++) {
        const int row = 8 * (2 * w + j) + (l >> 3);
        const int chunk = (l & 7) ^ ((row >> 1) & 7);

        koff[j] = 2u * (row * 64 + 8 * chunk);
        voff[j] = 2u * (row * Npk + 8 * chunk);
    }
    const unsigned lds_k = (unsigned)(uintptr_t)&Ks[0][0][0] + 2048u * wu,
                   lds_v = (unsigned)(uintptr_t)&Vt[0][0][0] + 2048u * wu;
    /* Byte offsets of this lane's MFMA operand fragments within one slot:
     * K rows 32 c + kperm(l32) (c adds 4096 B), V^T rows l32 and 32 + l32
     * (+4096 B); the swizzle depends only on row bits 1..3, which c and
     * the +32 leave alone. */
    unsigned kro[4], vro[4];
    for (int i = 0; i < 4; i++) {
        kro[i] = 2u * (krow * 64 + swz(krow, 2 * i + h));
        vro[i] = 2u * (l32 * 64 + swz(l32, 2 * i + h));
    }
    const char *Kb = (const char *)&Ks[0][0][0], *Vb = (const char *)&Vt[0][0][0];

    const uint16_t *Qu = q16 + unit * Np * 64;
    const uint16_t *Ku = k16 + unit * Npk * 64;
    const uint16_t *Vu = vt16 + unit * 64 * Npk;
    const float *kn = knorm + unit * nblk;
    const int qi = tile * 128 + w * 32 + l32;
    /* A wave whose 32 queries all lie past N (the second half of a
     * 64-query tail tile) still fills its share of the K / V staging and
     * meets every barrier, but issues no MFMA or softmax work, leaving its
     * SIMD to the co-resident waves. */
    const bool idle = tile * 128 + __builtin_amdgcn_readfirstlane(w) * 32 >= N;
    /* This lane's row of the additive bias table (exp2 domain, -inf past
     * Nk), if any; queries past N read the last row (never stored). */
    const int bH = d.bW > 0 ? Nk / d.bW : 0;
    const float *brow = EXT && d.bias
                            ? d.bias + ((long)unit * N + (qi < N ? qi : N - 1)) *
                                           (d.bW > 0 ? bH + d.bW : Npk)
                            : nullptr;
    bf16x8 qb[4];
    SoftState st;
    float qn; /* |q| of this lane's query, rounded up */
    bool shifted = false; /* some lane's m != 0 */

    /* Async copy of block kb into `slot`: wave w, pass j fills LDS rows
     * 8 (2 w + j) .. +7; lane i lands on row + i / 8, physical chunk
     * i % 8, so it fetches logical chunk (i % 8) ^ ((row >> 1) & 7). The
     * per-lane byte offsets do not depend on the block; the bases (block
     * start in global memory, destination rows in LDS) are wave-uniform
     * and live in SGPRs. */
    auto load_block = [&](int kb, int slot) {
        const uint16_t *kb_ = Ku + (long)kb * 64 * 64, *vb_ = Vu + kb * 64;

        for (int j = 0; j < 2; j++) {
            g2lds16_s(kb_, koff[j], lds_k + 8192u * slot + 1024u * j);
            g2lds16_s(vb_, voff[j], lds_v + 8192u * slot + 1024u * j);
        }
    };
    /* The first block of the plain instance: K's two copies before V's,
     * so that its Q K^T waits for K's only (the block loop below). Later
     * blocks keep K and V interleaved (K's copies first measured 2 % slower
     * on the balanced launch's global block). */
    auto load_first = [&](int kb, int slot) {
        if constexpr (!SK) {
            const uint16_t *kb_ = Ku + (long)kb * 64 * 64, *vb_ = Vu + kb * 64;

            for (int j = 0; j < 2; j++)
                g2lds16_s(kb_, koff[j], lds_k + 8192u * slot + 1024u * j);
            for (int j = 0; j < 2; j++)
                g2lds16_s(vb_, voff[j], lds_v + 8192u * slot + 1024u * j);
        }
        else
            load_block(kb, slot);
    };
    float kn_next = kn[kb0];

    /* Q through LDS (not in the bias / causal instance, whose registers
     * it would spill): the wave's 32 query rows (128 B each) go to slot 1
     * (free until the first barrier; rows 32 w .. +31 of a 128-row area,
     * Ks[1] then Vt[1]) by four whole-row copies with K's swizzle, then
     * into the MFMA B fragments: row l32, logical chunk 2 s + h. A direct
     * load per fragment touches 32 rows at 32 bytes each per instruction,
     * four instructions per line, in the start-up burst of every
     * workgroup (windowed 15.82 -> 15.62 us). Rows past Np read row
     * Np - 1 (never stored). */
    if constexpr (!EXT) {
        const unsigned qlds = (unsigned)(uintptr_t)(wu < 2 ? &Ks[1][32 * wu][0]
                                                           : &Vt[1][32 * (wu - 2)][0]);

        for (int j = 0; j < 4; j++) {
            const int row = 32 * w + 8 * j + (l >> 3), chunk = (l & 7) ^ ((row >> 1) & 7);
            const int qrow = tile * 128 + row < Np ? tile * 128 + row : Np - 1;

            g2lds16_s(Qu, 2u * ((unsigned)qrow * 64u + 8u * chunk), qlds + 1024u * j);
        }
        load_first(kb0, 0);
        /* The Q copies landed (the block's four may still be in flight). */
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");

        const char *qa = wu < 2 ? (const char *)&Ks[1][32 * wu][0]
                                : (const char *)&Vt[1][32 * (wu - 2)][0];

        for (int s = 0; s < 4; s++)
            qb[s] = *(const bf16x8 *)(qa + 128 * l32 + 2 * swz(l32, 2 * s + h));
    }
    else {
        load_block(kb0, 0);
        for (int s = 0; s < 4; s++) {
            if (qi < Np)
                qb[s] = *(const bf16x8 *)(Qu + (long)qi * 64 + 16 * s + 8 * h);
            else
                for (int e = 0; e < 8; e++)
                    qb[s][e] = (__bf16)0.0f;
        }
    }
    qn = 0.0f;
    for (int s = 0; s < 4; s++)
        for (int e = 0; e < 8; e++)
            qn = fmaf((float)qb[s][e], (float)qb[s][e], qn);
    qn = sqrtf(qn + __shfl_xor(qn, 32, 64)) * (1.0f + 0x1p-10f);
    for (int r = 0; r < 16; r++) {
        st.o0[r] = 0.0f;
        st.o1[r] = 0.0f;
    }
    st.m = 0.0f;
    st.l = 0.0f;

    /* Unrolled by two so that the slot is a constant: the LDS fragment
     * addresses are then one register plus an immediate offset. The first
     * block (`first_c`; not in the bias / causal instance, whose Q loads
     * wait for everything before it, nor in the balanced launch's, where
     * it measured 0.5 % slower) is split: its barrier waits for the
     * K copies only (the four copies of the block are this wave's
     * youngest loads, K's first: load_first), and a second barrier after
     * the softmax for the V^T copies, which arrive while the first Q K^T
     * runs. */
    auto block = [&](int kb, auto slot_c, auto first_c) {
        constexpr int slot = decltype(slot_c)::value;
        constexpr bool split = decltype(first_c)::value && !EXT && !SK;
        bf16x8 kf[8], vf[8], pb[4];
        f32x16 s0, s1;
        /* Can this block's scores exceed m + SAFE_SPAN for some lane? */
        const bool check =
            __ballot(brow || qn * kn_next - st.m > SAFE_SPAN) != 0;

        if constexpr (split)
            asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        /* Next block's bound, loaded after the barrier so that its latency
         * hides behind this block rather than in the barrier's wait. */
        kn_next = kn[kb + 1 < kb1 ? kb + 1 : kb];
        if (kb + 1 < kb1)
            load_block(kb + 1, slot ^ 1);
        /* Split first block: this wave's V^T copies land (the next block's
         * four, if issued, are younger), then every wave's. */
        auto v_landed = [&]() {
            if (kb + 1 < kb1)
                asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        };
        auto load_vf = [&]() {
            for (int t4 = 0; t4 < 4; t4++) {
                vf[2 * t4] = *(const bf16x8 *)(Vb + 8192 * slot + vro[t4]);
                if (!H32)
                    vf[2 * t4 + 1] = *(const bf16x8 *)(Vb + 8192 * slot + 4096 + vro[t4]);
            }
        };
        if (idle) {
            if constexpr (split)
                v_landed();
            return;
        }
        /* Head width 32 (H32): channels 32..63 of the packed operands are
         * zero, so only the first two 16-channel steps of Q K^T and the
         * first 32 output channels of P V carry work. */
        for (int c = 0; c < 2; c++)
            for (int ds = 0; ds < (H32 ? 2 : 4); ds++)
                kf[4 * c + ds] = *(const bf16x8 *)(Kb + 8192 * slot + 4096 * c + kro[ds]);
        if constexpr (!split)
            load_vf();
        /* Both 32-key halves at once: two independent Q K^T chains. */
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[0], qb[0], zero16, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[4], qb[0], zero16, 0, 0, 0);
        for (int ds = 1; ds < (H32 ? 2 : 4); ds++) {
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ds], qb[ds], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[4 + ds], qb[ds], s1, 0, 0, 0);
        }
        if (shifted)
            for (int r = 0; r < 16; r++) {
                s0[r] -= st.m;
                s1[r] -= st.m;
            }
        if (kb * 64 + 64 > Nk)
            for (int r = 0; r < 16; r++) {
                const int key = kb * 64 + 16 * (r >> 3) + 8 * h + (r & 7);

                s0[r] += key < Nk ? 0.0f : -INFINITY;
                s1[r] += key + 32 < Nk ? 0.0f : -INFINITY;
            }
        if (EXT && brow) {
            /* Additive box bias in the exp2 domain (no bound on it: every
             * such block takes the exact max below). Registers 8a .. 8a + 7
             * of s0 are keys 16 a + 8 h .. +7 of the block, s1's 32
             * further. */
            /* Rows at head width 32 only: at 64 the instance has no
             * registers to spare for them (they spilled 20 VGPRs). */
            if (H32 && d.bW > 0) {
                const int yb = kb * 64 / d.bW, xb = kb * 64 - yb * d.bW;

                for (int a = 0; a < 2; a++) {
                    int y, x;

                    block_yx(yb, xb, d.bW, 16 * a + 8 * h, y, x);
                    box_add<8>(brow, bH, Nk, kb * 64 + 16 * a + 8 * h, y, x, s0, 8 * a);
                    block_yx(yb, xb, d.bW, 32 + 16 * a + 8 * h, y, x);
                    box_add<8>(brow, bH, Nk, kb * 64 + 32 + 16 * a + 8 * h, y, x, s1, 8 * a);
                }
            }
            else {
                const float *bk = brow + kb * 64 + 8 * h;

                for (int a = 0; a < 2; a++) {
                    const f32x4 b0 = *(const f32x4 *)(bk + 16 * a);
                    const f32x4 b1 = *(const f32x4 *)(bk + 16 * a + 4);
                    const f32x4 b2 = *(const f32x4 *)(bk + 32 + 16 * a);
                    const f32x4 b3 = *(const f32x4 *)(bk + 32 + 16 * a + 4);

                    for (int e = 0; e < 4; e++) {
                        s0[8 * a + e] += b0[e];
                        s0[8 * a + 4 + e] += b1[e];
                        s1[8 * a + e] += b2[e];
                        s1[8 * a + 4 + e] += b3[e];
                    }
                }
            }
        }
        if (EXT && d.causal)
            for (int r = 0; r < 16; r++) {
                const int key = kb * 64 + 16 * (r >> 3) + 8 * h + (r & 7);

                s0[r] += key > qi ? -INFINITY : 0.0f;
                s1[r] += key + 32 > qi ? -INFINITY : 0.0f;
            }
        if (check) {
            /* Exact block max relative to m, decided per query (lanes l
             * and l ^ 32 share it): m moves up to a block max past
             * m + SAFE_SPAN, rescaling O and l by at most 1; it moves down
             * only while the query has no weight yet (l = 0, so O = 0 and
             * nothing is rescaled) and its block max lies below
             * m - SAFE_SPAN, so that its first weights do not underflow. A
             * query whose keys are all masked in this block stays put. */
            float mx = max16(s1, max16(s0, -INFINITY));

            mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32, 64));
            const bool empty = st.l + __shfl_xor(st.l, 32, 64) == 0.0f;
            const float mv = mx > SAFE_SPAN ||
                                     (empty && mx < -SAFE_SPAN && mx != -INFINITY)
                                 ? mx
                                 : 0.0f;

            if (__ballot(mv != 0.0f) != 0) {
                const float corr = __builtin_amdgcn_exp2f(-__builtin_fmaxf(mv, 0.0f));

                st.l *= corr;
                for (int r = 0; r < 16; r++) {
                    st.o0[r] *= corr;
                    st.o1[r] *= corr;
                    s0[r] -= mv;
                    s1[r] -= mv;
                }
                st.m += mv;
                shifted = true;
            }
        }
        for (int r = 0; r < 16; r++) {
            s0[r] = __builtin_amdgcn_exp2f(s0[r]);
            s1[r] = __builtin_amdgcn_exp2f(s1[r]);
        }
        for (int a = 0; a < 2; a++)
            for (int e = 0; e < 8; e++) {
                pb[a][e] = (__bf16)s0[8 * a + e];
                pb[2 + a][e] = (__bf16)s1[8 * a + e];
            }
        if constexpr (split) {
            v_landed();
            load_vf();
        }
        for (int t4 = 0; t4 < 4; t4++) {
            st.o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[2 * t4], pb[t4], st.o0, 0, 0, 0);
            if (!H32)
                st.o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[2 * t4 + 1], pb[t4], st.o1, 0, 0, 0);
        }
        st.l += sum32(s0, s1);
    };
    int lvl = -1;

    /* The plain instance peels the first pair (its first block split);
     * the others keep one loop (a peeled copy of the block spills
     * registers in the balanced launch's instance). */
    int kbs = kb0;

    if constexpr (!EXT && !SK) {
        prio_by_progress(pdone, ptotal, lvl);
        if (kb0 < kb1)
            block(kb0, std::integral_constant<int, 0>(), std::true_type());
        if (kb0 + 1 < kb1)
            block(kb0 + 1, std::integral_constant<int, 1>(), std::false_type());
        kbs = kb0 + 2;
    }
    for (int kb = kbs; kb < kb1; kb += 2) {
        prio_by_progress(pdone + kb - kb0, ptotal, lvl);
        block(kb, std::integral_constant<int, 0>(), std::false_type());
        if (kb + 1 < kb1)
            block(kb + 1, std::integral_constant<int, 1>(), std::false_type());
    }
    __builtin_amdgcn_s_setprio(0);

    if (SK && (kb0 > 0 || kb1 < nblk)) {
        /* A piece of a tile cut between workgroups: leave this piece's
         * per-lane state (O, m, l; 34 floats, lane-minor) in the record
         * of (workgroup, first or last piece), count it in, and let the
         * last piece to arrive merge all pieces in piece order (the same
         * bits whichever arrives last) and store the tile. The pieces of
         * a tile come from the stream-K
         * workgroups of its XCD whose ranges meet its key blocks in that
         * XCD's list of R shared (tile, key block) pairs, whose first tile
         * is rbase; `rank` is the workgroup's record owner index, XCD
         * G + its index among the XCD's G stream-K workgroups.
         *
         * Records and counters are only touched by agent-scope relaxed
         * atomics, which go to the device's coherent memory rather than
         * an XCD's L2; waiting for the record stores to complete
         * (vmcnt(0)) before the count orders them without the L2
         * write-back and invalidate of a device-scope fence, which cost
         * far more than the kernel itself when every workgroup issues
         * them. */
        const int tid = (int)unit * ntiles + tile, t0 = (tid - rbase) * nblk;
        /* An XCD whose remainder has fewer pairs than sk.G workgroups
         * uses one per pair. */
        const int G = R < sk.G ? R : sk.G, xg = (int)rank / sk.G * sk.G, me = (int)rank - xg;
        auto owner = [&](int idx) { return (int)((((unsigned)idx + 1) * (unsigned)G - 1) / (unsigned)R); };
        auto start = [&](int r) { return (int)((unsigned)r * (unsigned)R / (unsigned)G); };
        auto slot_of = [&](int r) { return 2 * (xg + r) + (start(r) < t0 ? 1 : 0); };
        const int r0 = owner(t0), r1 = owner(t0 + nblk - 1);
        float *rec = sk.rec + ((long)slot_of(me) * 4 + w) * 34 * 64 + l;

        auto put = [&](int k, float v) {
            __hip_atomic_store(rec + 64 * k, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        };
        for (int r = 0; r < 16; r++) {
            put(r, st.o0[r]);
            put(16 + r, st.o1[r]);
        }
        put(32, st.m);
        put(33, st.l);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (t == 0)
            arrived = __hip_atomic_fetch_add(&sk.cnt[tid], 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (arrived != (unsigned)(r1 - r0))
            return;
        if (t == 0)
            __hip_atomic_store(&sk.cnt[tid], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        /* The merge does not depend on which piece arrived last: the
         * pieces are folded in piece order r0 .. r1 into a running (M, L,
         * O), as the online softmax folds blocks (O and L rescaled by
         * 2^(M_old - M) when M grows, the piece added with weight
         * 2^(m_r - M)), this piece's own state (the bits of its record) at
         * its own place. One wait on memory per other piece, its 34 loads
         * in flight together. (The pieces' largest m read first, then the
         * sums: one more wait, 1.7 % on the global ViT block; holding two
         * records at once spills in this instance.) */
        auto rec_of = [&](int r) {
            return sk.rec + ((long)slot_of(r) * 4 + w) * 34 * 64 + l;
        };
        auto get = [&](const float *pr, int k) {
            return __hip_atomic_load(pr + 64 * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        };
        f32x16 a0 = zero16, a1 = zero16;
        float L = 0.0f, M = -INFINITY;

        for (int r = r0; r <= r1; r++) {
            f32x16 p0, p1;
            float pm, pl;

            if (r == me) {
                p0 = st.o0;
                p1 = st.o1;
                pm = st.m;
                pl = st.l;
            }
            else {
                const float *pr = rec_of(r);

                for (int r2 = 0; r2 < 16; r2++) {
                    p0[r2] = get(pr, r2);
                    p1[r2] = get(pr, 16 + r2);
                }
                pm = get(pr, 32);
                pl = get(pr, 33);
            }
            const float Mn = __builtin_fmaxf(M, pm);
            const float ca = __builtin_amdgcn_exp2f(M - Mn), cp = __builtin_amdgcn_exp2f(pm - Mn);

            for (int r2 = 0; r2 < 16; r2++) {
                a0[r2] = fmaf(p0[r2], cp, a0[r2] * ca);
                a1[r2] = fmaf(p1[r2], cp, a1[r2] * ca);
            }
            L = fmaf(pl, cp, L * ca);
            M = Mn;
        }
        st.o0 = a0;
        st.o1 = a1;
        st.l = L;
        st.m = M;
    }
    st.l += __shfl_xor(st.l, 32, 64);
    if constexpr (SPL) {
        if (!split_merge<!H32>(part, sk.cnt, unit * ntiles + tile, nsplit, sp, !idle, st.o0,
                               st.o1, st.m, st.l))
            return;
    }
    /* Final O / l. */
    const float inv = 1.0f / st.l;
    const long b0 = unit / d.nb1, b1 = unit % d.nb1;
    void *const Obuf = d.O;
    const long obase = d.ooff + b0 * d.so0 + b1 * d.so1;
    const int ldo = d.ldo, ocols = d.hd;
    const bool f32out = d.odt == DT_F32;

    if ((((obase | (long)ldo) & (f32out ? 3 : 7)) | ((uintptr_t)Obuf & 15)) == 0) {
        /* Output rows 16-byte aligned: transpose the wave's O^T through
         * LDS so that 8 lanes write one 128-byte line of one query row.
         * The slot of block kb1 - 2 (or the unused one) is free: every
         * wave passed the last barrier after its final reads of it. Each
         * wave takes 4 KB; 16-byte chunk c of staging row r sits at chunk
         * c ^ (r & 7), which keeps both the writes (8 rows, one chunk)
         * and the reads (one row, 8 chunks) free of bank conflicts. */
        const int fs = (kb1 - kb0) & 1;
        char *stg = w < 2 ? (char *)&Ks[fs][32 * w][0] : (char *)&Vt[fs][32 * (w - 2)][0];
        /* The lane index again, opaque to the compiler: the staging
         * offsets below are then formed here rather than kept from the
         * prologue across the key loop (which spilled them). */
        int l = threadIdx.x & 63;

        asm volatile("" : "+v"(l));
        const int l32 = l & 31, h = l >> 5;
        const int q0 = qi - l32, c = l & 7;
        /* All 32 rows of the wave inside N (every wave but those of a
         * ragged tail tile): the stores need no per-row test. */
        const bool full = q0 + 32 <= N;

        if (f32out) {
            /* Two passes of 32 columns (128 B per row); one for hd 32. The
             * four staged chunks are read before any is stored, so their
             * LDS latencies overlap instead of one per store. */
            for (int half = 0; half < ocols / 32; half++) {
                const f32x16 &o = half ? st.o1 : st.o0;
                f32x4 v[4];

                for (int g = 0; g < 4; g++) {
                    const f32x4 x = {o[4 * g] * inv, o[4 * g + 1] * inv,
                                     o[4 * g + 2] * inv, o[4 * g + 3] * inv};

                    *(f32x4 *)(stg + 128 * l32 + 16 * ((2 * g + h) ^ (l32 & 7))) = x;
                }
                for (int j = 0; j < 4; j++) {
                    const int row = 8 * j + (l >> 3);

                    v[j] = *(const f32x4 *)(stg + 128 * row + 16 * (c ^ (row & 7)));
                }
                float *ob = (float *)Obuf + obase + (long)(q0 + (l >> 3)) * ldo + 32 * half + 4 * c;

                if (full)
                    for (int j = 0; j < 4; j++)
                        __builtin_nontemporal_store(v[j], (f32x4 *)(ob + (long)8 * j * ldo));
                else
                    for (int j = 0; j < 4; j++)
                        if (q0 + 8 * j + (l >> 3) < N)
                            __builtin_nontemporal_store(v[j], (f32x4 *)(ob + (long)8 * j * ldo));
            }
        }
        else {
            /* One pass: a row is 64 bf16 = 128 B; lane (l32, h) holds
             * columns 8 g + 4 h .. +3, half h of logical chunk g. */
            for (int g = 0; g < 8; g++) {
                const f32x16 &o = g < 4 ? st.o0 : st.o1;
                const int r = 4 * (g & 3);
                const uint2 pk = {pack_bf16x2(o[r] * inv, o[r + 1] * inv),
                                  pack_bf16x2(o[r + 2] * inv, o[r + 3] * inv)};

                *(uint2 *)(stg + 128 * l32 + 16 * (g ^ (l32 & 7)) + 8 * h) = pk;
            }
            u32x4 v[4];

            for (int j = 0; j < 4; j++) {
                const int row = 8 * j + (l >> 3);

                v[j] = *(const u32x4 *)(stg + 128 * row + 16 * (c ^ (row & 7)));
            }
            uint16_t *ob = (uint16_t *)Obuf + obase + (long)(q0 + (l >> 3)) * ldo + 8 * c;

            if (8 * c < ocols) {
                if (full)
                    for (int j = 0; j < 4; j++)
                        *(u32x4 *)(ob + (long)8 * j * ldo) = v[j];
                else
                    for (int j = 0; j < 4; j++)
                        if (q0 + 8 * j + (l >> 3) < N)
                            *(u32x4 *)(ob + (long)8 * j * ldo) = v[j];
            }
        }
    }
    else if (qi < N) {
        const long orow = obase + (long)qi * ldo;
        const bool wide = ocols > 32;

        if (f32out) {
            for (int r = 0; r < 16; r++) {
                const int dd = 8 * (r >> 2) + 4 * h + (r & 3);

                ((float *)Obuf)[orow + dd] = st.o0[r] * inv;
                if (wide)
                    ((float *)Obuf)[orow + 32 + dd] = st.o1[r] * inv;
            }
        }
        else {
            for (int r = 0; r < 16; r++) {
                const int dd = 8 * (r >> 2) + 4 * h + (r & 3);

                ((uint16_t *)Obuf)[orow + dd] = f2bf(st.o0[r] * inv);
                if (wide)
                    ((uint16_t *)Obuf)[orow + 32 + dd] = f2bf(st.o1[r] * inv);
            }
        }
    }
}

template <bool EXT, bool H32, bool SK, bool SPL>
__global__ __launch_bounds__(256, 3) void k_attn_bf16(attn_desc d,
                                                      const uint16_t *__restrict__ q16,
                                                      const uint16_t *__restrict__ k16,
                                                      const uint16_t *__restrict__ vt16,
                                                      const float *__restrict__ knorm,
                                                      float *__restrict__ part,
                                                      int nsplit, sk_desc sk)
{
    const int nblk = (d.Nk + 63) / 64, ntiles = (d.N + 127) / 128;
    /* XCD-aware order: workgroups are dispatched to the XCDs round-robin,
     * so workgroup g runs on XCD g % NXCD; give each XCD a contiguous run
     * of work, i.e. whole units, whose K / V then stay in that XCD's L2
     * instead of every XCD streaming every unit. */
    const unsigned per_xcd = gridDim.x / NXCD;
    const unsigned rank = (blockIdx.x % NXCD) * per_xcd + blockIdx.x / NXCD;

    if (!SK) {
        /* One (unit, query tile, key split) item per workgroup: split sp
         * takes key blocks [sp nblk / nsplit, (sp + 1) nblk / nsplit); with
         * nsplit > 1 (SPL) the splits merge inside the launch. 32-bit item
         * arithmetic (the launcher keeps the grid below 2^31). */
        const unsigned total = (unsigned)d.nb * ntiles * nsplit, item = rank;

        if (item >= total)
            return;
        const unsigned us = nsplit > 1 ? item / (unsigned)nsplit : item;
        const int sp = (int)(item - us * (unsigned)nsplit);
        const long unit = us / (unsigned)ntiles;
        const int tile = (int)(us - (unsigned)unit * (unsigned)ntiles);

        const int kb0 = (int)((long)sp * nblk / nsplit), kb1 = (int)((long)(sp + 1) * nblk / nsplit);

        attn_tile<EXT, H32, false, SPL>(d, q16, k16, vt16, knorm, part, nsplit, sp, sk, rank,
                                        unit, tile, kb0, kb1, 0, kb1 - kb0, 0, 0);
        return;
    }
    /* Balanced launch (sk_desc): XCD x (workgroup g runs on XCD g % NXCD)
     * owns tiles [x per, x per + nx), per = total / NXCD rounded up; its
     * workgroups j < dp take whole tiles, its G further ones (j = dp + s)
     * share the R key blocks of its remaining tiles, [s R / G, (s + 1) R /
     * G) each, tile after tile; a tile cut between them is finished by the
     * piece that arrives last. 32-bit arithmetic: the launcher keeps R G
     * below 2^31. A barrier between segments keeps the next segment's
     * first copies out of LDS the last one still reads. */
    const unsigned total = (unsigned)d.nb * ntiles, per = (total + NXCD - 1) / NXCD;
    const unsigned x = blockIdx.x % NXCD, j = blockIdx.x / NXCD;
    const int tx0 = (int)(x * per);
    const int nx = total > x * per ? (int)(total - x * per < per ? total - x * per : per) : 0;

    const bool whole = (int)j < sk.dp;
    const int sidx = (int)j - sk.dp, rbase = tx0 + sk.dp, R = (nx - sk.dp) * nblk;
    /* Stream-K workgroups of this XCD: one per pair if it has fewer
     * pairs left than sk.G (the last XCD's share may be short). */
    const int G = R < sk.G ? R : sk.G;

    if (whole ? (int)j >= nx : sidx >= G || R <= 0)
        return;
    /* A whole-tile workgroup is a stream-K range of one uncut tile (no
     * record), so that both kinds share one instance of the tile body. */
    const int a0 = whole ? ((int)j - sk.dp) * nblk
                         : (int)((unsigned)sidx * (unsigned)R / (unsigned)G);
    const int b = whole ? a0 + nblk : (int)(((unsigned)sidx + 1) * (unsigned)R / (unsigned)G);
    int a = a0;

    while (a < b) {
        const int tl = a / nblk, tid = rbase + tl;
        const int k0 = a - tl * nblk;
        const int k1 = k0 + (b - a) < nblk ? k0 + (b - a) : nblk;
        /* The descriptor read afresh in each segment, through an opaque
         * copy of its kernel-argument address (d is the first argument,
         * at offset 0): otherwise the compiler hoists every field the
         * epilogue reads out of the segment loop and holds them in SGPRs
         * across the key loop, which then spills. */
        typedef const __attribute__((address_space(4))) attn_desc kdesc;
        kdesc *dp = (kdesc *)__builtin_amdgcn_kernarg_segment_ptr();

        asm volatile("" : "+s"(dp));
        attn_tile<EXT, H32, true, false>(*dp, q16, k16, vt16, knorm, part, 1, 0, sk,
                                  x * (unsigned)sk.G + (unsigned)sidx, tid / ntiles, tid % ntiles,
                                  k0, k1, a - a0, b - a0, rbase, R);
        a += k1 - k0;
        if (a < b)
            __syncthreads();
    }
}

/* Launch-starved shapes (one 576-token window: 16 units of 9 key blocks)
 * in one launch: a workgroup of NG WPG waves takes 32 WPG queries of one
 * unit, and its NG groups of WPG waves take NG contiguous ranges of the
 * key blocks (double-buffered K / V^T slots per group), in lockstep: each
 * iteration's barrier serves every group, a group past its last block
 * only meets the barriers. The groups then meet in LDS: groups 1 .. NG -
 * 1 leave their per-lane (O^T, m, l), and group 0 scales every group's
 * (O, l) to the largest m and sums them in group order (the same bits
 * every launch) before storing O / l. Block body and softmax reference
 * point as k_attn_bf16's (plain instance: head width 64, no bias, no
 * causal mask). With RES (at most RESB key blocks) every key block of
 * the unit stays resident in LDS: each group's copies are all issued at
 * the start, and iteration i waits only for the copies of its group's
 * block i (the younger ones may still fly), so no block waits for a
 * copy issued one block earlier. */
#define RESB 9
template <int NG, int WPG, bool RES>
__global__ __launch_bounds__(64 * NG * WPG) void k_attn_bf16_grp(attn_desc d,
                                                               const uint16_t *__restrict__ q16,
                                                               const uint16_t *__restrict__ k16,
                                                               const uint16_t *__restrict__ vt16,
                                                               const float *__restrict__ knorm)
{
    constexpr int QT = 32 * WPG, CPW = 16 / WPG; /* queries per tile, copies per wave */
    /* Double-buffered: [group][slot][K, V^T][row][64 bf16], 32 KiB per
     * group. Resident: [key block][K, V^T][row][64] plus 4 KiB of output
     * staging per group-0 wave. */
    constexpr int LDSB = RES ? RESB * 16384 + 4096 * WPG : NG * 32768;
    __shared__ __attribute__((aligned(16))) char KV[LDSB];
    const int t = threadIdx.x, l = t & 63, h = l >> 5, l32 = l & 31;
    const int wu = __builtin_amdgcn_readfirstlane(t >> 6), g = wu / WPG, wl = wu - g * WPG;
    const int N = d.N, Nk = d.Nk, Np = (N + 63) / 64 * 64, Npk = (Nk + 63) / 64 * 64,
              nblk = Npk / 64;
    const int ntiles = (N + QT - 1) / QT;
    const long unit = blockIdx.x / ntiles;
    const int tile = (int)(blockIdx.x - unit * ntiles);
    const int kb0 = g * nblk / NG, kb1 = (g + 1) * nblk / NG, iters = (nblk + NG - 1) / NG;
    const int qi = tile * QT + wl * 32 + l32;
    const bool idle = tile * QT + wl * 32 >= N;
    const uint16_t *Ku = k16 + unit * Npk * 64, *Vu = vt16 + unit * 64 * Npk;
    const float *kn = knorm + unit * nblk;
    const int krow = kperm(l32);
    const f32x16 zero16 = {};
    const char *base = KV + (RES ? 0 : 32768 * g);
    const unsigned lds_g = (unsigned)(uintptr_t)base;
    unsigned goffk[CPW], goffv[CPW], ldso[CPW];
    bool isk[CPW];

    /* Copy c = wl CPW + j of the group's 16 per block: K rows (c < 8) or
     * V^T rows (c >= 8) 8 (c % 8) .. +7; lane i lands on row + i / 8,
     * physical chunk i % 8, logical chunk (i % 8) ^ ((row >> 1) & 7). */
    for (int j = 0; j < CPW; j++) {
        const int c = wl * CPW + j, row = 8 * (c & 7) + (l >> 3);
        const int chunk = (l & 7) ^ ((row >> 1) & 7);

        isk[j] = c < 8;
        goffk[j] = 2u * ((unsigned)row * 64u + 8u * chunk);
        goffv[j] = 2u * ((unsigned)row * (unsigned)Npk + 8u * chunk);
        ldso[j] = (c < 8 ? 0u : 8192u) + 1024u * (c & 7);
    }
    /* Copies of block kb into 16 KiB area `area` of the group's LDS. */
    auto load_block = [&](int kb, int area) {
        for (int j = 0; j < CPW; j++) {
            if (isk[j])
                g2lds16_s(Ku + (long)kb * 64 * 64, goffk[j], lds_g + 16384u * area + ldso[j]);
            else
                g2lds16_s(Vu + kb * 64, goffv[j], lds_g + 16384u * area + ldso[j]);
        }
    };
    unsigned kro[4], vro[4];
    for (int i = 0; i < 4; i++) {
        kro[i] = 2u * (krow * 64 + swz(krow, 2 * i + h));
        vro[i] = 2u * (l32 * 64 + swz(l32, 2 * i + h));
    }
    bf16x8 qb[4];
    SoftState st;
    float qn;
    bool shifted = false;
    {
        const int qr = qi < Np ? qi : Np - 1;
        const uint16_t *Qr = q16 + (unit * Np + qr) * 64;

        for (int s = 0; s < 4; s++)
            qb[s] = *(const bf16x8 *)(Qr + 16 * s + 8 * h);
    }
    if constexpr (RES) {
        for (int kb = kb0; kb < kb1; kb++)
            load_block(kb, kb);
    }
    else if (kb0 < kb1)
        load_block(kb0, 0);
    qn = 0.0f;
    for (int s = 0; s < 4; s++)
        for (int e = 0; e < 8; e++)
            qn = fmaf((float)qb[s][e], (float)qb[s][e], qn);
    qn = sqrtf(qn + __shfl_xor(qn, 32, 64)) * (1.0f + 0x1p-10f);
    for (int r = 0; r < 16; r++) {
        st.o0[r] = 0.0f;
        st.o1[r] = 0.0f;
    }
    st.m = 0.0f;
    st.l = 0.0f;

    for (int it = 0; it < iters; it++) {
        const int kb = kb0 + it, slot = it & 1;
        const bool active = kb < kb1;
        const float kbound = active ? kn[kb] : 0.0f;

        if constexpr (RES) {
            /* This wave's copies of the group's later blocks may fly. */
            const int later = kb1 - 1 - kb;

            if (later >= 2)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * CPW) : "memory");
            else if (later == 1)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CPW) : "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (!RES && kb + 1 < kb1)
            load_block(kb + 1, slot ^ 1);
        if (!active || idle)
            continue;
        const char *Kb = base + 16384 * (RES ? kb : slot), *Vb = Kb + 8192;
        bf16x8 kf[8], vf[8], pb[4];
        f32x16 s0, s1;
        const bool check = __ballot(qn * kbound - st.m > SAFE_SPAN) != 0;

        for (int c = 0; c < 2; c++)
            for (int ds = 0; ds < 4; ds++)
                kf[4 * c + ds] = *(const bf16x8 *)(Kb + 4096 * c + kro[ds]);
        for (int t4 = 0; t4 < 4; t4++) {
            vf[2 * t4] = *(const bf16x8 *)(Vb + vro[t4]);
            vf[2 * t4 + 1] = *(const bf16x8 *)(Vb + 4096 + vro[t4]);
        }
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[0], qb[0], zero16, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[4], qb[0], zero16, 0, 0, 0);
        for (int ds = 1; ds < 4; ds++) {
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ds], qb[ds], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[4 + ds], qb[ds], s1, 0, 0, 0);
        }
        if (shifted)
            for (int r = 0; r < 16; r++) {
                s0[r] -= st.m;
                s1[r] -= st.m;
            }
        if (kb * 64 + 64 > Nk)
            for (int r = 0; r < 16; r++) {
                const int key = kb * 64 + 16 * (r >> 3) + 8 * h + (r & 7);

                s0[r] += key < Nk ? 0.0f : -INFINITY;
                s1[r] += key + 32 < Nk ? 0.0f : -INFINITY;
            }
        if (check) {
            float mx = max16(s1, max16(s0, -INFINITY));

            mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32, 64));
            const bool empty = st.l + __shfl_xor(st.l, 32, 64) == 0.0f;
            const float mv = mx > SAFE_SPAN || (empty && mx < -SAFE_SPAN && mx != -INFINITY)
                                 ? mx
                                 : 0.0f;

            if (__ballot(mv != 0.0f) != 0) {
                const float corr = __builtin_amdgcn_exp2f(-__builtin_fmaxf(mv, 0.0f));

                st.l *= corr;
                for (int r = 0; r < 16; r++) {
                    st.o0[r] *= corr;
                    st.o1[r] *= corr;
                    s0[r] -= mv;
                    s1[r] -= mv;
                }
                st.m += mv;
                shifted = true;
            }
        }
        for (int r = 0; r < 16; r++) {
            s0[r] = __builtin_amdgcn_exp2f(s0[r]);
            s1[r] = __builtin_amdgcn_exp2f(s1[r]);
        }
        for (int a = 0; a < 2; a++)
            for (int e = 0; e < 8; e++) {
                pb[a][e] = (__bf16)s0[8 * a + e];
                pb[2 + a][e] = (__bf16)s1[8 * a + e];
            }
        for (int t4 = 0; t4 < 4; t4++) {
            st.o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[2 * t4], pb[t4], st.o0, 0, 0, 0);
            st.o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[2 * t4 + 1], pb[t4], st.o1, 0, 0, 0);
        }
        st.l += sum32(s0, s1);
    }

    /* Groups 1 .. NG - 1 leave (O^T, m, l) per lane (34 floats, lane-minor)
     * in the freed slots; group 0 merges them in group order. */
    __syncthreads();
    float *ex = (float *)KV;
    if (g > 0) {
        float *rec = ex + ((g - 1) * WPG + wl) * 34 * 64 + l;

        for (int r = 0; r < 16; r++) {
            rec[64 * r] = st.o0[r];
            rec[64 * (16 + r)] = st.o1[r];
        }
        rec[64 * 32] = st.m;
        rec[64 * 33] = st.l;
    }
    __syncthreads();
    if (g > 0 || idle)
        return;
    float M = st.m;

    for (int gg = 1; gg < NG; gg++)
        M = __builtin_fmaxf(M, ex[((gg - 1) * WPG + wl) * 34 * 64 + 64 * 32 + l]);
    {
        const float c0 = __builtin_amdgcn_exp2f(st.m - M);

        for (int r = 0; r < 16; r++) {
            st.o0[r] *= c0;
            st.o1[r] *= c0;
        }
        st.l *= c0;
    }
    for (int gg = 1; gg < NG; gg++) {
        const float *rec = ex + ((gg - 1) * WPG + wl) * 34 * 64 + l;
        const float c = __builtin_amdgcn_exp2f(rec[64 * 32] - M);

        for (int r = 0; r < 16; r++) {
            st.o0[r] = fmaf(rec[64 * r], c, st.o0[r]);
            st.o1[r] = fmaf(rec[64 * (16 + r)], c, st.o1[r]);
        }
        st.l = fmaf(rec[64 * 33], c, st.l);
    }
    st.l += __shfl_xor(st.l, 32, 64);
    const float inv = 1.0f / st.l;
    const long b0 = unit / d.nb1, b1 = unit % d.nb1;
    const long obase = d.ooff + b0 * d.so0 + b1 * d.so1;
    const bool f32out = d.odt == DT_F32;

    if ((((obase | (long)d.ldo) & (f32out ? 3 : 7)) | ((uintptr_t)d.O & 15)) == 0) {
        /* Rows 16-byte aligned: O^T transposed through a 4 KiB staging area
         * per wave at the end of LDS (past the groups' records), 16-byte
         * chunk c of staging row r at chunk c ^ (r & 7); 8 lanes write one
         * 128-byte line of a query row. */
        char *stg = KV + LDSB - 4096 * (WPG - wl);
        const int q0 = qi - l32, c = l & 7;

        if (f32out) {
            for (int half = 0; half < 2; half++) {
                const f32x16 &o = half ? st.o1 : st.o0;
                f32x4 v[4];

                for (int gq = 0; gq < 4; gq++) {
                    const f32x4 x = {o[4 * gq] * inv, o[4 * gq + 1] * inv, o[4 * gq + 2] * inv,
                                     o[4 * gq + 3] * inv};

                    *(f32x4 *)(stg + 128 * l32 + 16 * ((2 * gq + h) ^ (l32 & 7))) = x;
                }
                for (int j = 0; j < 4; j++) {
                    const int row = 8 * j + (l >> 3);

                    v[j] = *(const f32x4 *)(stg + 128 * row + 16 * (c ^ (row & 7)));
                }
                float *ob = (float *)d.O + obase + (long)(q0 + (l >> 3)) * d.ldo + 32 * half + 4 * c;

                for (int j = 0; j < 4; j++)
                    if (q0 + 8 * j + (l >> 3) < N)
                        *(f32x4 *)(ob + (long)8 * j * d.ldo) = v[j];
            }
        }
        else {
            for (int gq = 0; gq < 8; gq++) {
                const f32x16 &o = gq < 4 ? st.o0 : st.o1;
                const int r = 4 * (gq & 3);
                const uint2 pk = {pack_bf16x2(o[r] * inv, o[r + 1] * inv),
                                  pack_bf16x2(o[r + 2] * inv, o[r + 3] * inv)};

                *(uint2 *)(stg + 128 * l32 + 16 * (gq ^ (l32 & 7)) + 8 * h) = pk;
            }
            u32x4 v[4];

            for (int j = 0; j < 4; j++) {
                const int row = 8 * j + (l >> 3);

                v[j] = *(const u32x4 *)(stg + 128 * row + 16 * (c ^ (row & 7)));
            }
            uint16_t *ob = (uint16_t *)d.O + obase + (long)(q0 + (l >> 3)) * d.ldo + 8 * c;

            for (int j = 0; j < 4; j++)
                if (q0 + 8 * j + (l >> 3) < N)
                    *(u32x4 *)(ob + (long)8 * j * d.ldo) = v[j];
        }
        return;
    }
    if (qi >= N)
        return;
    const long orow = obase + (long)qi * d.ldo;

    for (int r = 0; r < 16; r++) {
        const int dd = 8 * (r >> 2) + 4 * h + (r & 3);

        if (d.odt == DT_F32) {
            ((float *)d.O)[orow + dd] = st.o0[r] * inv;
            ((float *)d.O)[orow + 32 + dd] = st.o1[r] * inv;
        }
        else {
            ((uint16_t *)d.O)[orow + dd] = f2bf(st.o0[r] * inv);
            ((uint16_t *)d.O)[orow + 32 + dd] = f2bf(st.o1[r] * inv);
        }
    }
}

/* ng key groups (4: 64-query tiles of 2 waves per group; 2: 128-query
 * tiles of 4 waves per group); plain attention of head width 64. */
extern "C" int launch_attn_bf16_grp(const attn_desc *d, const void *q16, const void *k16,
                                    const void *vt16, const float *knorm, int ng, void *stream)
{
    const int nblk = (d->Nk + 63) / 64, qt = ng == 4 ? 64 : 128;
    const long grid = (long)d->nb * ((d->N + qt - 1) / qt);

    if ((ng != 2 && ng != 4) || nblk < ng || d->Nk < 1 || d->N < 1 || d->hd != 64 ||
        d->bias || d->causal || grid > 0x7fffffffL)
        return hipErrorInvalidConfiguration;
    if (ng == 4 && nblk <= RESB)
        hipLaunchKernelGGL((k_attn_bf16_grp<4, 2, true>), dim3((unsigned)grid), dim3(512), 0,
                           (hipStream_t)stream, *d, (const uint16_t *)q16, (const uint16_t *)k16,
                           (const uint16_t *)vt16, knorm);
    else if (ng == 4)
        hipLaunchKernelGGL((k_attn_bf16_grp<4, 2, false>), dim3((unsigned)grid), dim3(512), 0,
                           (hipStream_t)stream, *d, (const uint16_t *)q16, (const uint16_t *)k16,
                           (const uint16_t *)vt16, knorm);
    else
        hipLaunchKernelGGL((k_attn_bf16_grp<2, 4, false>), dim3((unsigned)grid), dim3(512), 0,
                           (hipStream_t)stream, *d, (const uint16_t *)q16, (const uint16_t *)k16,
                           (const uint16_t *)vt16, knorm);
    return hipGetLastError();
}

/* Zero fill of the balanced attention's arrival counters (a kernel, not
 * a memset, so that it may sit in a captured graph). */
__global__ __launch_bounds__(256) void k_attn_sk_zero(unsigned *cnt, long n)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;

    if (i < n)
        cnt[i] = 0u;
}

extern "C" int launch_attn_sk_zero(unsigned *cnt, long n, void *stream)
{
    if (n < 1 || (n + 255) / 256 > 0x7fffffffL)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_attn_sk_zero, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, cnt, n);
    return hipGetLastError();
}

extern "C" int launch_attn_bf16(const attn_desc *d, const void *q16,
                                const void *k16, const void *vt16,
                                const float *knorm, float *part, int nsplit,
                                float *skrec, unsigned *skcnt, int skG, int skdp,
                                void *stream)
{
    const int nblk = (d->Nk + 63) / 64;
    const long tiles = (long)d->nb * ((d->N + 127) / 128);
    const long total = tiles * nsplit, per = (tiles + NXCD - 1) / NXCD;
    const long grid = skG ? (long)NXCD * (skdp + skG) : (total + NXCD - 1) / NXCD * NXCD;
    const sk_desc sk = {skrec, skcnt, skG, skdp};

    /* Key splits merge inside the launch: their records in part (nb,
     * 128-query tiles, SPLIT_RECS(nsplit) records of 9216 floats) and
     * SPLIT_CNT arrival counts per tile in skcnt. */
    if (grid > 0x7fffffffL || d->Nk < 1 || nsplit < 1 || nsplit > nblk || nsplit > 64 ||
        (nsplit > 1 && (!part || !skcnt)))
        return hipErrorInvalidConfiguration;
    /* Balanced launch: whole-key tiles, head width 64 without bias or
     * causal mask, some tiles left over on an XCD after dp whole ones and
     * at least one shared key block per stream-K workgroup, both buffers
     * given, 32-bit pair arithmetic. */
    if (skG && (nsplit != 1 || skG < 0 || skdp < 0 || per <= skdp ||
                (per - skdp) * nblk < skG || (per - skdp) * nblk * skG > 0x7fffffffL ||
                !skrec || !skcnt || d->bias || d->causal || d->hd != 64))
        return hipErrorInvalidConfiguration;
    {
        const bool ext = d->bias || d->causal, h32 = d->hd == 32;
        auto kern = skG ? k_attn_bf16<false, false, true, false>
                    : nsplit > 1
                        ? (ext ? (h32 ? k_attn_bf16<true, true, false, true>
                                      : k_attn_bf16<true, false, false, true>)
                               : (h32 ? k_attn_bf16<false, true, false, true>
                                      : k_attn_bf16<false, false, false, true>))
                        : (ext ? (h32 ? k_attn_bf16<true, true, false, false>
                                      : k_attn_bf16<true, false, false, false>)
                               : (h32 ? k_attn_bf16<false, true, false, false>
                                      : k_attn_bf16<false, false, false, false>));

        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, *d,
                           (const uint16_t *)q16, (const uint16_t *)k16,
                           (const uint16_t *)vt16, knorm, part, nsplit, sk);
    }
    return hipGetLastError();
}

extern "C" int launch_attn_f32(const attn_desc *d, float *part, unsigned *cnt, int nsplit,
                               void *stream)
{
    const int nblk = (d->Nk + 31) / 32;
    const long total = (long)d->nb * ((d->N + 127) / 128) * nsplit;
    const long grid = (total + NXCD - 1) / NXCD * NXCD;
    const bool ext = d->causal || d->bias;

    if (d->N < 1 || d->nb < 1 || grid > 0x7fffffffL || d->Nk < 1 || nsplit < 1 || nsplit > 64 ||
        nsplit > nblk || (nsplit > 1 && (!part || !cnt)) || (d->hd != 64 && d->hd != 32) ||
        (d->hd == 32 && d->rope))
        return hipErrorInvalidConfiguration;
    {
        auto kern = nsplit > 1 ? (d->hd == 32 ? (ext ? k_attn_f32<32, true, true>
                                                     : k_attn_f32<32, false, true>)
                                              : (ext ? k_attn_f32<64, true, true>
                                                     : k_attn_f32<64, false, true>))
                               : (d->hd == 32 ? (ext ? k_attn_f32<32, true, false>
                                                     : k_attn_f32<32, false, false>)
                                              : (ext ? k_attn_f32<64, true, false>
                                                     : k_attn_f32<64, false, false>));

        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, *d,
                           part, cnt, nsplit);
    }
    return hipGetLastError();
}
