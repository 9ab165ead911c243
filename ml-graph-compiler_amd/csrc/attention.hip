// Fused scaled-dot-product attention: O = softmax(scale * Q K^T) V for every (batch, head).
//
// The reference runs the head split, QK^T, the scale, the softmax, PV and the head merge as
// separate nodes (MatMul -> Mul -> Softmax -> MatMul with Transposes around them, as the
// transformer sample builds it: src/ml_graph_compiler/samples.py:178-245), each a pass over
// memory. This kernel reads Q, K and V through strides straight out of the fused QKV
// projection output and writes O in the [batch, seq, head * dim] layout of the head merge,
// so the score matrix and the transposed copies never reach HBM.
//
// One workgroup of 256 threads (4 waves) owns 64 query rows of one (batch, head) and streams
// the keys in blocks of 64 with a running ("online") softmax, so neither S nor Skv is bounded:
//  1. the Q rows go to LDS ([row][d], d contiguous) once;
//  2. per key block, K goes to LDS as [key][d] and V transposed as [d][key] from registers
//     loaded while the previous block was being multiplied (the next block's loads are issued
//     right after, so HBM latency is paid once per workgroup, not once per block); each wave
//     multiplies a 32x32 block of the scores with v_mfma_f32_32x32x2f32 and writes it, scaled,
//     biased and masked as the graph says, into an LDS tile;
//  3. four threads per row take the block's row maximum, raise the running maximum m, turn the
//     scores into exp(t - m), add them to the running sum l and publish exp(m_old - m);
//  4. each wave rescales its 32x32 block of O by that factor and accumulates P V on MFMA;
//  5. O is divided by l and leaves as 128-byte row segments.
// With a causal mask, key blocks that lie wholly past the diagonal hold only the fill value; they
// are skipped when their terms are exactly zero in fp32 (fill = -inf, or fill at least 110
// below every row's running maximum, where expf underflows to 0).
// Operand fragments follow the GEMM kernels' convention: within a 32-wide k chunk, lanes
// 0-31 take k 0..15 and lanes 32-63 take k 16..31 (the same permutation on both operands).
#include "mgc_device.h"

namespace mgc {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int ATT_BQ = 64;      // query rows per workgroup
constexpr int ATT_BK = 64;      // keys per block
constexpr int ATT_DMAX = 64;    // head dim limit
constexpr int ATT_P = ATT_DMAX + 4;    // row pitch (floats) of every LDS tile
constexpr float ATT_SKIP_MARGIN = 110.f;

struct AttnDev {
    int B, H, S, Skv, D;
    const float *q, *k, *v;
    long q_b, q_s, q_h, k_b, k_s, k_h, v_b, v_s, v_h;
    float *o;
    long o_b, o_s, o_h;
    float scale;
    int scale_div;
    const float *bias;
    long bias_b, bias_h, bias_s, bias_j;
    const unsigned char *mask;
    long mask_b, mask_h, mask_s, mask_j;
    int mask_keep;
    int causal;
    float fill;
};

template <int G>
__global__ void __launch_bounds__(256 * G) attention_kernel(const AttnDev p) {
    __shared__ __attribute__((aligned(16))) float Qs[ATT_BQ * ATT_P];
    __shared__ __attribute__((aligned(16))) float Ks_all[G][ATT_BK * ATT_P];
    __shared__ __attribute__((aligned(16))) float Vt_all[G][ATT_DMAX * ATT_P];  // [d][key]
    __shared__ __attribute__((aligned(16))) float Ps_all[G][ATT_BQ * ATT_P];    // scores, then exp terms
    __shared__ float rowscale_all[G][ATT_BQ];  // exp(m_old - m_new) of the block; 1 / l at the end
    __shared__ float mstate[G][2][ATT_BQ];     // G > 1: each group's final m and l per row

    const int tid = threadIdx.x;
    const int grp = G > 1 ? tid >> 8 : 0;  // key group: takes key blocks grp, grp + G, ...
    const int gt = tid & 255;              // thread within its group
    float *const Ks = Ks_all[grp];
    float *const Vt = Vt_all[grp];
    float *const Ps = Ps_all[grp];
    float *const rowscale = rowscale_all[grp];
    const int lane = gt & 63;
    const int wave = gt >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 31, lh = lane >> 5;
    const int qblocks = (p.S + ATT_BQ - 1) / ATT_BQ;
    // XCD order: the query blocks of one (batch, head) run on one XCD, so its K and V come
    // into that XCD's L2 once instead of once per query block
    const int blk = xcd_block();
    const int bh = blk / qblocks;
    const int q0 = (blk - bh * qblocks) * ATT_BQ;
    const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
    const float *qbase = p.q + b * p.q_b + h * p.q_h;
    const float *kbase = p.k + b * p.k_b + h * p.k_h;
    const float *vbase = p.v + b * p.v_b + h * p.v_h;
    const float *bias = p.bias ? p.bias + b * p.bias_b + h * p.bias_h : nullptr;
    const unsigned char *mask = p.mask ? p.mask + b * p.mask_b + h * p.mask_h : nullptr;
    const int D = p.D, D4 = p.D >> 2;
    const int kblocks = (p.Skv + ATT_BK - 1) / ATT_BK;
    const int dchunks = (D + 31) >> 5;
    const int q_last = min(q0 + ATT_BQ, p.S) - 1;
    const float scale = p.scale, fill = p.fill;
    const bool scale_div = p.scale_div != 0, causal = p.causal != 0, keep_set = p.mask_keep != 0;
    const float NEG_INF = -__builtin_huge_valf();
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
    // softmax role: four neighbouring threads share a row
    const int srow = gt >> 2, part = gt & 3;
    float m_run = NEG_INF, l_run = 0.f;

    // Tiles of 64 rows x 16 float quads are moved as 4 quads per thread. Q and K: thread t takes
    // row e >> 4, quad e & 15 of e = t + 256 i (16 lanes read one row's 256 contiguous bytes).
    // V: row e & 63, quad e >> 6, so a wave's 64 lanes hold 64 consecutive keys of one quad and
    // the transposed LDS stores [d][key] hit 64 consecutive words (no bank conflicts).
    constexpr int QUADS = ATT_BQ * (ATT_DMAX / 4) / 256;
    static_assert(ATT_BQ == ATT_BK && QUADS == 4, "tile moves assume 64 x 64 tiles");
    f4 kst[QUADS], vst[QUADS];
    // Issue the global loads of key block k0 into registers (zero past Skv and past D); they
    // stay in flight while the current block is multiplied.
    auto load_kv = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < QUADS; ++i) {
            const int e = gt + 256 * i;
            const int r = e >> 4, c4 = e & 15;
            kst[i] = zero4;
            if (k0 + r < p.Skv && c4 < D4) kst[i] = *reinterpret_cast<const f4 *>(kbase + (long)(k0 + r) * p.k_s + c4 * 4);
            const int rv = e & 63, cv = e >> 6;
            vst[i] = zero4;
            if (k0 + rv < p.Skv && cv < D4) vst[i] = *reinterpret_cast<const f4 *>(vbase + (long)(k0 + rv) * p.v_s + cv * 4);
        }
    };
    auto store_kv = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < QUADS; ++i) {
            const int e = gt + 256 * i;
            *reinterpret_cast<f4 *>(&Ks[(e >> 4) * ATT_P + (e & 15) * 4]) = kst[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) Vt[((e >> 6) * 4 + j) * ATT_P + (e & 63)] = vst[i][j];
        }
    };

    // 1. Q rows (rows past S and columns past D are zero), requested with the first key block
    {
        f4 qst[QUADS];
        if (grp == 0) {
#pragma unroll
            for (int i = 0; i < QUADS; ++i) {
                const int e = gt + 256 * i;
                const int r = e >> 4, c4 = e & 15;
                qst[i] = zero4;
                if (q0 + r < p.S && c4 < D4) qst[i] = *reinterpret_cast<const f4 *>(qbase + (long)(q0 + r) * p.q_s + c4 * 4);
            }
        }
        if (grp < kblocks) load_kv(grp * ATT_BK);
        if (grp == 0) {
#pragma unroll
            for (int i = 0; i < QUADS; ++i) {
                const int e = gt + 256 * i;
                *reinterpret_cast<f4 *>(&Qs[(e >> 4) * ATT_P + (e & 15) * 4]) = qst[i];
            }
        }
    }

    floatx16 oacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[r] = 0.f;

    // Each iteration every group takes its own key block (none when past the keys); barriers are
    // workgroup-wide, so a group without a block still meets them.
    const int iters = (kblocks + G - 1) / G;
    for (int it = 0; it < iters; ++it) {
        const int kb = it * G + grp;
        const int k0 = kb * ATT_BK;
        bool active = kb < kblocks;
        if (G == 1) {
            if (causal && k0 > q_last) {
                // every key from here on is masked in every row of the block
                const bool zero_terms = q0 + srow > q_last || fill == NEG_INF || fill <= m_run - ATT_SKIP_MARGIN;
                if (__syncthreads_and(zero_terms)) break;
            }
        } else if (active && causal && k0 > q_last && fill == NEG_INF) {
            active = false;  // every term of this block is exactly zero
        }
        __syncthreads();  // Ks, Vt, Ps and rowscale free; Qs visible
        // 2. K block [key][d], V block transposed [d][key], from the registers loaded one block
        // ahead; then the next block's loads go out
        if (kb < kblocks) store_kv();
        if (kb + G < kblocks) load_kv(k0 + G * ATT_BK);
        __syncthreads();
        floatx16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        if (active) {
            for (int c = 0; c < dchunks; ++c) {
                f4 af[4], bf[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    af[s] = *reinterpret_cast<const f4 *>(&Qs[(wm * 32 + li) * ATT_P + c * 32 + lh * 16 + 4 * s]);
                    bf[s] = *reinterpret_cast<const f4 *>(&Ks[(wn * 32 + li) * ATT_P + c * 32 + lh * 16 + 4 * s]);
                }
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s][e], bf[s][e], acc, 0, 0, 0);
            }
            // register r of lane (li, lh): query row 8 (r / 4) + 4 lh + r % 4, key column li
            const int key = k0 + wn * 32 + li;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
                const int q = q0 + row;
                float t;
                if (key >= p.Skv) {
                    t = NEG_INF;
                } else if (q >= p.S) {
                    t = 0.f;
                } else {
                    t = scale_div ? acc[r] / scale : acc[r] * scale;
                    if (bias) t += bias[(long)q * p.bias_s + (long)key * p.bias_j];
                    bool keep = true;
                    if (causal) keep = key <= q;
                    else if (mask) keep = (mask[(long)q * p.mask_s + (long)key * p.mask_j] != 0) == keep_set;
                    if (!keep) t = fill;
                }
                Ps[row * ATT_P + wn * 32 + li] = t;
            }
        }
        __syncthreads();

        // 3. running softmax over the block's 64 scores of each row (16 per thread)
        if (active) {
            float *prow = &Ps[srow * ATT_P + part * 16];
            f4 x[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) x[c] = *reinterpret_cast<const f4 *>(prow + 4 * c);
            float bm = NEG_INF;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) bm = fmaxf(bm, x[c][e]);
            bm = fmaxf(bm, __shfl_xor(bm, 1, 64));
            bm = fmaxf(bm, __shfl_xor(bm, 2, 64));
            const float m_new = fmaxf(m_run, bm);
            const float alpha = m_new == NEG_INF ? 1.f : expf(m_run - m_new);
            float sum = 0.f;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float pe = x[c][e] == NEG_INF ? 0.f : expf(x[c][e] - m_new);
                    x[c][e] = pe;
                    sum += pe;
                }
                *reinterpret_cast<f4 *>(prow + 4 * c) = x[c];
            }
            sum += __shfl_xor(sum, 1, 64);
            sum += __shfl_xor(sum, 2, 64);
            l_run = l_run * alpha + sum;
            m_run = m_new;
            if (part == 0) rowscale[srow] = alpha;
        }
        __syncthreads();

        // 4. O = alpha O + P V for this block (V^T in LDS: [d][key])
        if (active && wn * 32 < D) {
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[r] *= rowscale[wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3)];
#pragma unroll
            for (int c = 0; c < ATT_BK / 32; ++c) {
                f4 af[4], bf[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    af[s] = *reinterpret_cast<const f4 *>(&Ps[(wm * 32 + li) * ATT_P + c * 32 + lh * 16 + 4 * s]);
                    bf[s] = *reinterpret_cast<const f4 *>(&Vt[(wn * 32 + li) * ATT_P + c * 32 + lh * 16 + 4 * s]);
                }
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        oacc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s][e], bf[s][e], oacc, 0, 0, 0);
            }
        }
    }
    __syncthreads();  // every wave is past its last read of rowscale
    const int d = wn * 32 + li;
    if (G == 1) {
        if (part == 0) rowscale[srow] = 1.0f / l_run;
    } else {
        // The groups' partial states combine as m = max(m_g), l = sum_g l_g exp(m_g - m),
        // O = sum_g O_g exp(m_g - m) / l. Groups past the first leave m, l and O (in their Ps
        // tile) in LDS; the first group scales and adds.
        if (part == 0) {
            mstate[grp][0][srow] = m_run;
            mstate[grp][1][srow] = l_run;
        }
        if (grp > 0 && d < D) {
#pragma unroll
            for (int r = 0; r < 16; ++r) Ps[(wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3)) * ATT_P + d] = oacc[r];
        }
        __syncthreads();
        if (grp == 0 && part == 0) {
            float m = NEG_INF;
#pragma unroll
            for (int g2 = 0; g2 < G; ++g2) m = fmaxf(m, mstate[g2][0][srow]);
            float l = 0.f;
#pragma unroll
            for (int g2 = 0; g2 < G; ++g2) {
                const float mg = mstate[g2][0][srow];
                const float w = mg == NEG_INF ? 0.f : expf(mg - m);
                mstate[g2][0][srow] = w;  // the group's weight
                l += mstate[g2][1][srow] * w;
            }
            rowscale[srow] = 1.0f / l;
        }
        __syncthreads();
        if (grp == 0 && d < D) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
                float v = oacc[r] * mstate[0][0][row];
#pragma unroll
                for (int g2 = 1; g2 < G; ++g2) v += Ps_all[g2][row * ATT_P + d] * mstate[g2][0][row];
                oacc[r] = v;
            }
        }
    }
    __syncthreads();

    // 5. O rows: register r of lane (li, lh) is query 8 (r / 4) + 4 lh + r % 4, column d = li
    if (grp == 0 && d < D) {
        float *obase = p.o + b * p.o_b + h * p.o_h + d;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
            const int q = q0 + row;
            if (q < p.S) obase[(long)q * p.o_s] = oacc[r] * rowscale[row];
        }
    }
}

// Attention over at most 32 W keys (W <= 4) in one pass, for short sequences (BERT-base's 128
// keys): one workgroup of W waves per (batch, head, 32 queries), wave w owning keys 32 w ..
// 32 w + 31. No running softmax:
//  1. every global load goes out at once, all 16 bytes wide: wave w's share of the 32 query rows
//     (rows w, w + W, ...), its 32 key rows (lane (li, lh) takes d = 32 c + 16 lh .. + 15 of key
//     row li) and its 32 V rows; the query rows meet in LDS (each read from memory once per
//     workgroup) and each wave's V rows go to an LDS tile of its own, from which the P V
//     products read V by column;
//  2. S^T = K Q^T on v_mfma_f32_32x32x2f32 (keys as rows, queries as columns), so register r of
//     lane (li, lh) holds the score of key 8 (r / 4) + 4 lh + r % 4 and query li;
//  3. the scores are scaled, biased and masked as the graph says, each query's maximum is taken
//     over the lane pair (li, li + 32) and, through LDS, over the waves, and the scores become
//     exp(t - m);
//  4. O^T = V^T P^T: the score registers already are the B operand of this product (register r
//     gives keys 8 (r / 4) + 4 lh + r % 4 of lane half lh, and the A operand takes V at the same
//     keys), so P never goes through LDS;
//  5. waves 1 .. W - 1 leave their O^T partials (in their own V tiles) and row sums in LDS;
//     wave 0 adds them in wave order, divides by the sum and writes each query's D outputs.
// Terms are exp(t - m) with m the maximum over all keys (fp32 expf, as the streaming kernel),
// and keys past Skv add nothing.
template <int W, bool HAS_BIAS, bool HAS_MASK>
__global__ void __launch_bounds__(64 * W) attention_short_kernel(const AttnDev p, int vec_out) {
    constexpr int QP = 68;  // query tile pitch: the 16 rows one 16-byte read covers hit different banks
    constexpr int VP = 72;  // V tile pitch: keys 4 apart (the two lane halves) land 32 banks apart
    __shared__ float wmax[W][32];
    __shared__ float wsum[W][32];
    __shared__ __attribute__((aligned(16))) float qs[32 * QP];
    __shared__ __attribute__((aligned(16))) float vs[W][32 * VP];  // later: the waves' O^T partials

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, lh = lane >> 5;
    const int qblocks = (p.S + 31) >> 5;
    // XCD order: the query blocks of one (batch, head) run on one XCD, so its K and V come
    // into that XCD's L2 once instead of once per query block
    const int blk = xcd_block();
    const int bh = blk / qblocks;
    const int q0 = (blk - bh * qblocks) * 32;
    const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
    const float *qbase = p.q + b * p.q_b + h * p.q_h;
    const float *kbase = p.k + b * p.k_b + h * p.k_h;
    const float *vbase = p.v + b * p.v_b + h * p.v_h;
    const float *bias = p.bias ? p.bias + b * p.bias_b + h * p.bias_h : nullptr;
    const unsigned char *mask = p.mask ? p.mask + b * p.mask_b + h * p.mask_h : nullptr;
    const int D = p.D;
    const float NEG_INF = -__builtin_huge_valf();
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const int q = q0 + li;
    const int k0 = 32 * w;

    // 1. operands. Buffer loads: an element past S, Skv or D gets an offset past the resource's
    // end and reads as zero, so the loads need no branches and the multiplies wait only for their
    // own.
    constexpr unsigned OOB = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        (void *)qbase, (short)0, (int)(((long)(p.S - 1) * p.q_s + D) * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void *)kbase, (short)0, (int)(((long)(p.Skv - 1) * p.k_s + D) * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void *)vbase, (short)0, (int)(((long)(p.Skv - 1) * p.v_s + D) * 4), 0x00020000);
    // this wave's share of the 32 x 16 query quads: quads (w + W j) 64 + lane (row e / 16, d 4 (e % 16))
    constexpr int QL = 32 * 16 / (64 * W) > 0 ? 32 * 16 / (64 * W) : 1;  // 16-byte quads per lane
    f4 qv[QL];
#pragma unroll
    for (int j = 0; j < QL; ++j) {
        const int e = (w + W * j) * 64 + lane;  // quad e of the 32 x 16 query quads
        const int row = e >> 4, d = (e & 15) * 4;
        const unsigned o = e < 512 && q0 + row < p.S && d < D ? (unsigned)((long)(q0 + row) * p.q_s + d) * 4u : OOB;
        qv[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rq, o, 0, 0));
    }
    f4 kf[2][4];
    const bool q_ok = q < p.S, k_ok = k0 + li < p.Skv;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const int d = 32 * c + 16 * lh + 4 * s4;
            const unsigned ok = k_ok && d < D ? (unsigned)((long)(k0 + li) * p.k_s + d) * 4u : OOB;
            kf[c][s4] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rk, ok, 0, 0));
        }
    // this wave's 32 V rows: quad e = lane + 64 j of the 32 x 16 quads is row e / 16, d 4 (e % 16)
    f4 vq[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int e = lane + 64 * j;
        const int key = k0 + (e >> 4), d = (e & 15) * 4;
        const unsigned o = key < p.Skv && d < D ? (unsigned)((long)key * p.v_s + d) * 4u : OOB;
        vq[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rv, o, 0, 0));
    }

    // the additive bias and the mask of this lane's 16 scores (when the graph has them: HAS_BIAS,
    // HAS_MASK), requested with the operands; the addresses are clamped into the tensors and the
    // elements past S or Skv are not used
    const int qc = q_ok ? q : p.S - 1;
    float bv[16];
    unsigned char mv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int key = min(k0 + 8 * (r >> 2) + 4 * lh + (r & 3), p.Skv - 1);
        bv[r] = HAS_BIAS ? bias[(long)qc * p.bias_s + (long)key * p.bias_j] : 0.f;
        mv[r] = HAS_MASK ? mask[(long)qc * p.mask_s + (long)key * p.mask_j] : 0;
    }
    // every load above goes out before the first multiply (the scheduler would otherwise hold
    // some back to save registers and pay their latency one after another)
    __builtin_amdgcn_sched_barrier(0);

    // the query rows into LDS; once every wave's share is there, each lane takes d = 32 c +
    // 16 lh .. + 15 of query row li as the B operand
#pragma unroll
    for (int j = 0; j < QL; ++j) {
        const int e = (w + W * j) * 64 + lane;
        if (e < 512) *reinterpret_cast<f4 *>(&qs[(e >> 4) * QP + (e & 15) * 4]) = qv[j];
    }
    __syncthreads();
    f4 qf[2][4];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) qf[c][s4] = *reinterpret_cast<const f4 *>(&qs[li * QP + 32 * c + 16 * lh + 4 * s4]);

    // 2. S^T for this wave's 32 keys
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[c][s4][e], qf[c][s4][e], acc, 0, 0, 0);

    // this wave's V rows into its tile (read back by this wave only)
    float *const vt = vs[w];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int e = lane + 64 * j;
        *reinterpret_cast<f4 *>(&vt[(e >> 4) * VP + (e & 15) * 4]) = vq[j];
    }

    // 3. scores, the query's maximum over all keys, exp terms and this wave's sum
    const float scale = p.scale, fill = p.fill;
    const bool scale_div = p.scale_div != 0, causal = p.causal != 0, keep_set = p.mask_keep != 0;
    float m = NEG_INF;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int key = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
        float t;
        if (key >= p.Skv) {
            t = NEG_INF;
        } else if (!q_ok) {
            t = 0.f;
        } else {
            t = scale_div ? acc[r] / scale : acc[r] * scale;
            if (HAS_BIAS) t += bv[r];
            bool keep = true;
            if (causal) keep = key <= q;
            else if (HAS_MASK) keep = (mv[r] != 0) == keep_set;
            if (!keep) t = fill;
        }
        acc[r] = t;
        m = fmaxf(m, t);
    }
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    if (W > 1) {
        if (lh == 0) wmax[w][li] = m;
        __syncthreads();
#pragma unroll
        for (int w2 = 0; w2 < W; ++w2) m = w2 == 0 ? wmax[0][li] : fmaxf(m, wmax[w2][li]);
    }
    float l = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float pe = acc[r] == NEG_INF ? 0.f : expf(acc[r] - m);
        acc[r] = pe;
        l += pe;
    }
    l += __shfl_xor(l, 32, 64);

    // 4. O^T = V^T P^T over this wave's keys (the second d block only when D > 32)
    floatx16 o[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
    // V at key 8 (r / 4) + 4 lh + r % 4 (tile row) and d = 32 db + li
#pragma unroll
    for (int r = 0; r < 16; ++r)
        o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt[(8 * (r >> 2) + 4 * lh + (r & 3)) * VP + li], acc[r], o[0], 0, 0, 0);
    if (D > 32) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt[(8 * (r >> 2) + 4 * lh + (r & 3)) * VP + 32 + li], acc[r], o[1],
                                                       0, 0, 0);
    }

    // 5. wave order sum of the partials; register r of o[db] is d = 32 db + 8 (r / 4) + 4 lh + r % 4
    if (W > 1) {
        if (w > 0) {
            // into this wave's own V tile, whose last reads (this wave's P V operands) came before
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) vt[(16 * db + r) * 64 + lane] = o[db][r];
            if (lh == 0) wsum[w][li] = l;
        }
        __syncthreads();
        if (w > 0) return;
#pragma unroll
        for (int w2 = 1; w2 < W; ++w2) {
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[db][r] += vs[w2][(16 * db + r) * 64 + lane];
            l += wsum[w2][li];
        }
    }
    if (!q_ok) return;
    const float inv = 1.0f / l;
    float *orow = p.o + b * p.o_b + h * p.o_h + (long)q * p.o_s;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * db + 8 * g + 4 * lh;
            if (d >= D) continue;
            const f4 v = {o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv};
            if (vec_out) {
                *reinterpret_cast<f4 *>(orow + d) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) orow[d + e] = v[e];
            }
        }
}

}  // namespace mgc

using namespace mgc;

typedef void (*AttnShortKernel)(AttnDev, int);

extern "C" int mgc_hip_attention_supported(int S, int Skv, int D) {
    return S >= 1 && Skv >= 1 && D >= 4 && D <= ATT_DMAX && D % 4 == 0;
}

extern "C" void mgc_hip_attention(mgc_hip_exec *x, const mgc_hip_attention_args *a) {
    if (a->B <= 0 || a->H <= 0 || a->S <= 0) return;
    if (!mgc_hip_attention_supported(a->S, a->Skv, a->D)) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_attention: shape outside the kernel's limits", hipErrorInvalidValue);
        return;
    }
    const long blocks = (long)a->B * a->H * ((a->S + ATT_BQ - 1) / ATT_BQ);
    if (blocks > 0x7fffffffL) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_attention: grid too large", hipErrorInvalidValue);
        return;
    }
    AttnDev p;
    p.B = a->B;
    p.H = a->H;
    p.S = a->S;
    p.Skv = a->Skv;
    p.D = a->D;
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.q_b = a->q_b;
    p.q_s = a->q_s;
    p.q_h = a->q_h;
    p.k_b = a->k_b;
    p.k_s = a->k_s;
    p.k_h = a->k_h;
    p.v_b = a->v_b;
    p.v_s = a->v_s;
    p.v_h = a->v_h;
    p.o = a->o;
    p.o_b = a->o_b;
    p.o_s = a->o_s;
    p.o_h = a->o_h;
    p.scale = a->scale;
    p.scale_div = a->scale_div;
    {
        // dividing by a power of two equals multiplying by its (exact) reciprocal, bit for bit
        int ex = 0;
        const float mant = frexpf(a->scale, &ex);
        if (a->scale_div && mant == 0.5f && ex > -120 && ex < 120) {
            p.scale = ldexpf(1.0f, 1 - ex);
            p.scale_div = 0;
        }
    }
    p.bias = a->bias;
    p.bias_b = a->bias_b;
    p.bias_h = a->bias_h;
    p.bias_s = a->bias_s;
    p.bias_j = a->bias_j;
    p.mask = a->mask;
    p.mask_b = a->mask_b;
    p.mask_h = a->mask_h;
    p.mask_s = a->mask_s;
    p.mask_j = a->mask_j;
    p.mask_keep = a->mask_keep;
    p.causal = a->causal;
    p.fill = a->fill;
    // At most 128 keys: the one-pass kernel, a wave per 32 keys and a workgroup per 32 queries
    // (with eight waves its registers would no longer fit two waves per SIMD).
    if (a->Skv <= 128) {
        const long qb = (long)a->B * a->H * ((a->S + 31) / 32);
        const int vec_out = a->o_s % 4 == 0 && a->o_b % 4 == 0 && a->o_h % 4 == 0 && ((uintptr_t)a->o & 15) == 0;
        const int waves = (a->Skv + 31) / 32;
        if (qb <= 0x7fffffffL) {
            const int bm = (p.bias ? 1 : 0) | (p.mask && !p.causal ? 2 : 0);
            const int sel = (waves <= 1 ? 0 : waves <= 2 ? 1 : 2) * 4 + bm;
            static const AttnShortKernel table[12] = {
                &attention_short_kernel<1, false, false>, &attention_short_kernel<1, true, false>,
                &attention_short_kernel<1, false, true>,  &attention_short_kernel<1, true, true>,
                &attention_short_kernel<2, false, false>, &attention_short_kernel<2, true, false>,
                &attention_short_kernel<2, false, true>,  &attention_short_kernel<2, true, true>,
                &attention_short_kernel<4, false, false>, &attention_short_kernel<4, true, false>,
                &attention_short_kernel<4, false, true>,  &attention_short_kernel<4, true, true>};
            const int threads = 64 * (waves <= 1 ? 1 : waves <= 2 ? 2 : 4);
            MGC_LAUNCH(x, table[sel], dim3((unsigned)qb), dim3(threads), 0, p, vec_out);
            return;
        }
    }
    // Fewer (batch, head, 64-query) blocks than CUs and at least two key blocks: two groups of
    // four waves per workgroup take alternate key blocks and combine at the end (one workgroup
    // per CU then: the groups' tiles take 122 KB of LDS).
    const int kblocks = (a->Skv + ATT_BK - 1) / ATT_BK;
    if (blocks < 256 && kblocks >= 2)
        MGC_LAUNCH(x, attention_kernel<2>, dim3((unsigned)blocks), dim3(512), 0, p);
    else
        MGC_LAUNCH(x, attention_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, p);
}
