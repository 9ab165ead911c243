// Fused scaled-dot-product attention: O = softmax(scale * Q K^T) V for every (batch, head).
//
// The reference runs the head split, QK^T, the scale, the softmax, PV and the head merge as
// separate nodes (MatMul -> Mul -> Softmax -> MatMul with Transposes around them, as the
// transformer sample builds it: src/ml_graph_compiler/samples.py:178-245), each a pass over
// memory. This kernel reads Q, K and V through strides straight out of the fused QKV
// projection output and writes O in the [batch, seq, head * dim] layout of the head merge,
// so the score matrix and the transposed copies never reach HBM.
//
// One workgroup of 256 threads (4 waves) owns 64 query rows of one (batch, head):
//  1. the Q rows go to LDS ([row][d], d contiguous);
//  2. keys are taken 64 at a time; each wave multiplies a 32x32 block of the scores with
//     v_mfma_f32_32x32x2f32 and writes it, scaled, into an LDS score tile [64][keys];
//  3. four threads per row compute the row max, the exponentials and the sum, and leave the
//     normalized probabilities in the tile;
//  4. V is taken 64 keys at a time, transposed into LDS as [d][key], and each wave
//     accumulates a 32x32 block of O = P V; O leaves as 128-byte row segments.
// Operand fragments follow the GEMM kernels' convention: within a 32-wide k chunk, lanes
// 0-31 take k 0..15 and lanes 32-63 take k 16..31 (the same permutation on both operands).
#include "mgc_device.h"

namespace mgc {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int ATT_BQ = 64;      // query rows per workgroup
constexpr int ATT_BK = 64;      // keys per block
constexpr int ATT_DMAX = 64;    // head dim limit
constexpr int ATT_SMAX = 256;   // key count limit
constexpr int ATT_DP = ATT_DMAX + 4;         // row pitch of Q, K and V^T tiles
constexpr int ATT_SP = ATT_SMAX + 4;         // row pitch of the score tile

struct AttnDev {
    int B, H, S, Skv, D;
    const float *q, *k, *v;
    long q_b, q_s, q_h, k_b, k_s, k_h, v_b, v_s, v_h;
    float *o;
    long o_b, o_s, o_h;
    float scale;
};

__global__ void __launch_bounds__(256) attention_kernel(const AttnDev p) {
    __shared__ __attribute__((aligned(16))) float Qs[ATT_BQ * ATT_DP];
    __shared__ __attribute__((aligned(16))) float KVs[ATT_BK * ATT_DP];  // K block, then V^T block
    __shared__ __attribute__((aligned(16))) float Ss[ATT_BQ * ATT_SP];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 31, lh = lane >> 5;
    const int qblocks = (p.S + ATT_BQ - 1) / ATT_BQ;
    const int bh = blockIdx.x / qblocks;
    const int q0 = (blockIdx.x - bh * qblocks) * ATT_BQ;
    const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
    const float *qbase = p.q + b * p.q_b + h * p.q_h;
    const float *kbase = p.k + b * p.k_b + h * p.k_h;
    const float *vbase = p.v + b * p.v_b + h * p.v_h;
    const int D = p.D, D4 = p.D >> 2;
    const int kblocks = (p.Skv + ATT_BK - 1) / ATT_BK;
    const int dchunks = (D + 31) >> 5;
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};

    // 1. Q rows (rows past S and columns past D are zero)
    for (int e = tid; e < ATT_BQ * (ATT_DMAX / 4); e += 256) {
        const int r = e / (ATT_DMAX / 4), c4 = e - r * (ATT_DMAX / 4);
        f4 v = zero4;
        if (q0 + r < p.S && c4 < D4) v = *reinterpret_cast<const f4 *>(qbase + (long)(q0 + r) * p.q_s + c4 * 4);
        *reinterpret_cast<f4 *>(&Qs[r * ATT_DP + c4 * 4]) = v;
    }

    // 2. scores, one 64-key block at a time
    for (int kb = 0; kb < kblocks; ++kb) {
        __syncthreads();  // KVs free (previous block consumed), Qs visible
        for (int e = tid; e < ATT_BK * (ATT_DMAX / 4); e += 256) {
            const int r = e / (ATT_DMAX / 4), c4 = e - r * (ATT_DMAX / 4);
            const int key = kb * ATT_BK + r;
            f4 v = zero4;
            if (key < p.Skv && c4 < D4) v = *reinterpret_cast<const f4 *>(kbase + (long)key * p.k_s + c4 * 4);
            *reinterpret_cast<f4 *>(&KVs[r * ATT_DP + c4 * 4]) = v;
        }
        __syncthreads();
        floatx16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        for (int c = 0; c < dchunks; ++c) {
            f4 af[4], bf[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                af[s] = *reinterpret_cast<const f4 *>(&Qs[(wm * 32 + li) * ATT_DP + c * 32 + lh * 16 + 4 * s]);
                bf[s] = *reinterpret_cast<const f4 *>(&KVs[(wn * 32 + li) * ATT_DP + c * 32 + lh * 16 + 4 * s]);
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s][e], bf[s][e], acc, 0, 0, 0);
        }
        // register r of lane (li, lh): query row 8 (r / 4) + 4 lh + r % 4, key column li
        const int key = kb * ATT_BK + wn * 32 + li;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
            Ss[row * ATT_SP + key] = key < p.Skv ? acc[r] * p.scale : -__builtin_huge_valf();
        }
    }
    __syncthreads();

    // 3. softmax over each row's Skv scores: four neighbouring lanes share a row
    {
        const int row = tid >> 2, part = tid & 3;
        float *srow = &Ss[row * ATT_SP];
        const int ncol = kblocks * ATT_BK;
        float m = -__builtin_huge_valf();
        for (int j = part; j < ncol; j += 4) m = fmaxf(m, srow[j]);
        m = fmaxf(m, __shfl_xor(m, 1, 64));
        m = fmaxf(m, __shfl_xor(m, 2, 64));
        float sum = 0.f;
        for (int j = part; j < ncol; j += 4) {
            const float e = srow[j] == -__builtin_huge_valf() ? 0.f : expf(srow[j] - m);
            srow[j] = e;
            sum += e;
        }
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        const float inv = 1.0f / sum;
        for (int j = part; j < ncol; j += 4) srow[j] *= inv;
    }

    // 4. O = P V, one 64-key block of V at a time (V^T in LDS: [d][key])
    floatx16 oacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[r] = 0.f;
    for (int kb = 0; kb < kblocks; ++kb) {
        __syncthreads();  // probabilities written, KVs free
        for (int e = tid; e < ATT_BK * (ATT_DMAX / 4); e += 256) {
            const int r = e / (ATT_DMAX / 4), c4 = e - r * (ATT_DMAX / 4);
            const int key = kb * ATT_BK + r;
            f4 v = zero4;
            if (key < p.Skv && c4 < D4) v = *reinterpret_cast<const f4 *>(vbase + (long)key * p.v_s + c4 * 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) KVs[(c4 * 4 + j) * ATT_DP + r] = v[j];
        }
        __syncthreads();
        if (wn * 32 < D) {
#pragma unroll
            for (int c = 0; c < ATT_BK / 32; ++c) {
                f4 af[4], bf[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    af[s] = *reinterpret_cast<const f4 *>(&Ss[(wm * 32 + li) * ATT_SP + kb * ATT_BK + c * 32 + lh * 16 + 4 * s]);
                    bf[s] = *reinterpret_cast<const f4 *>(&KVs[(wn * 32 + li) * ATT_DP + c * 32 + lh * 16 + 4 * s]);
                }
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        oacc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s][e], bf[s][e], oacc, 0, 0, 0);
            }
        }
    }

    // 5. O rows: register r of lane (li, lh) is query 8 (r / 4) + 4 lh + r % 4, column d = li
    const int d = wn * 32 + li;
    if (d < D) {
        float *obase = p.o + b * p.o_b + h * p.o_h + d;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int q = q0 + wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
            if (q < p.S) obase[(long)q * p.o_s] = oacc[r];
        }
    }
}

}  // namespace mgc

using namespace mgc;

extern "C" int mgc_hip_attention_supported(int S, int Skv, int D) {
    return S >= 1 && Skv >= 1 && Skv <= ATT_SMAX && D >= 4 && D <= ATT_DMAX && D % 4 == 0;
}

extern "C" void mgc_hip_attention(mgc_hip_exec *x, const mgc_hip_attention_args *a) {
    if (a->B <= 0 || a->H <= 0 || a->S <= 0) return;
    if (!mgc_hip_attention_supported(a->S, a->Skv, a->D)) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_attention: shape outside the kernel's limits", hipErrorInvalidValue);
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
    const long blocks = (long)a->B * a->H * ((a->S + ATT_BQ - 1) / ATT_BQ);
    MGC_LAUNCH(x, attention_kernel, dim3((unsigned)blocks), dim3(256), 0, p);
}
