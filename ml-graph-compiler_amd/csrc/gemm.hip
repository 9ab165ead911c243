// fp32 GEMM and implicit-GEMM convolution on CDNA4 matrix cores (v_mfma_f32_32x32x2f32).
//
// Computes C[z] = act(alpha * A[z] B[z] + bias + beta * R[z]), the contract of the reference's
// mgc_gemm (src/ml_graph_compiler/codegen/runtime/mgc_kernels.c:282-396), with operands read as
// strided matrices or through implicit im2col of an NHWC (A) or NCHW (B) image.
//
// Design (MI355X-first, not a translation of the reference's Goto/BLIS CPU blocking):
//  * A workgroup of 256 threads (4 waves of 64) owns a BM x BN output tile; each wave owns a
//    WM x WN sub-tile made of 32x32 MFMA blocks, accumulated in 16 registers per block.
//  * K advances 32 at a time through double-buffered LDS. Both operands are stored k-contiguous
//    in LDS ([row][32 + 4 pad]) so every lane fetches its fragment with ds_read_b128.
//  * The 32x32x2 MFMA consumes two k per instruction, one per half-wave. The kernel assigns the
//    first 16 k of a stage to lanes 0-31 and the last 16 to lanes 32-63 (a permutation of the
//    summation order, applied identically to A and B), so each lane's 16 k values are
//    contiguous in LDS.
//  * Global loads are float4 (16 B) when the operand is k-contiguous (packed weights, NHWC
//    activations with channel counts divisible by 4) and branch-free (out-of-range lanes read
//    a valid address and select zero). Implicit im2col computes the (kh, kw, c) split of a
//    thread's k once per stage and reuses it for all of the thread's rows.
//  * The epilogue stages the accumulator tile through LDS, then every thread walks the tile in
//    16-byte chunks: coalesced float4 residual loads and stores, bias per float4, and one
//    activation dispatch per chunk. This keeps the kernel's code small (an unrolled per-register
//    epilogue would not fit the instruction cache) and its HBM traffic in full lines.
//  * The workgroup id is remapped so each of the 8 XCDs (each with its own L2) works on a
//    contiguous range of tiles, N fastest: tiles that share A rows share an L2.
//  * Small-M problems (the 128-row GEMM of the single-GEMM config) split K over extra
//    workgroups into a planner-provided workspace, then a reduction applies the epilogue.
#include "mgc_device.h"

namespace mgc {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));

enum { AM_VEC = 0, AM_CONV_VEC = 1, AM_GEN = 2 };
enum { BD_NK_VEC = 0, BD_KN_VEC = 1, BD_GEN = 2 };

struct GemmDev {
    int M, N, K;
    mgc_hip_operand a, b;
    float *c;
    long ldc;
    float alpha, beta;
    const float *bias;
    int bias_mode;
    const float *res;
    long ldr;
    int act;
    float lo, hi;
    int batch_rank;
    int bdims[4];
    long a_bs[4], b_bs[4], c_bs[4], r_bs[4];
    int split;    // K splits (1 = none)
    int kchunk;   // K per split, a multiple of 32
    float *ws;    // split partials [split][M][N]
    int tiles_m, tiles_n;
    int vec_out;  // 16-byte epilogue accesses are aligned (ldc, ldr, pointers)
};

__device__ __forceinline__ void batch_offsets(const GemmDev &p, int bz, long &ao, long &bo,
                                              long &co, long &ro) {
    ao = bo = co = ro = 0;
    int rem = bz;
#pragma unroll
    for (int d = 3; d >= 0; --d) {
        if (d < p.batch_rank) {
            int idx = rem % p.bdims[d];
            rem /= p.bdims[d];
            ao += idx * p.a_bs[d];
            bo += idx * p.b_bs[d];
            co += idx * p.c_bs[d];
            ro += idx * p.r_bs[d];
        }
    }
}

__device__ __forceinline__ f4 act4(f4 v, int act, float lo, float hi) {
    switch (act) {
    case MGC_ACT_RELU:
        v[0] = v[0] > 0.0f ? v[0] : 0.0f;
        v[1] = v[1] > 0.0f ? v[1] : 0.0f;
        v[2] = v[2] > 0.0f ? v[2] : 0.0f;
        v[3] = v[3] > 0.0f ? v[3] : 0.0f;
        return v;
    case MGC_ACT_CLIP:
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = fminf(fmaxf(v[e], lo), hi);
        return v;
    case MGC_ACT_GELU:
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gelu_erf_f(v[e]);
        return v;
    case MGC_ACT_GELU_TANH:
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gelu_tanh_f(v[e]);
        return v;
    case MGC_ACT_TANH:
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = tanh_f(v[e]);
        return v;
    case MGC_ACT_SIGMOID:
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = sigmoid_f(v[e]);
        return v;
    default: return v;
    }
}

template <int BM, int BN, int WGM, int AMODE, int BMODE>
__global__ void __launch_bounds__(256) gemm_mfma_kernel(const GemmDev p) {
    constexpr int BK = 32;
    constexpr int LDK = BK + 4;
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM;
    constexpr int WN = BN / WGN;
    constexpr int RM = WM / 32;
    constexpr int RN = WN / 32;
    static_assert(RM >= 1 && RN >= 1 && WGM * WGN == 4, "bad tile");
    constexpr int AV = BM / 32;  // float4 loads per thread per stage (vector A)
    constexpr int AG = BM / 8;   // scalar loads per thread per stage (generic A)
    constexpr int BV = BN / 32;
    constexpr int BG = BN / 8;
    constexpr int LDC = BN + 4;
    constexpr int SMEM_LOOP = 2 * (BM + BN) * LDK;
    constexpr int SMEM_EPI = BM * LDC;
    constexpr int SMEM = SMEM_LOOP > SMEM_EPI ? SMEM_LOOP : SMEM_EPI;

    __shared__ __attribute__((aligned(16))) float smem[SMEM];
    float *const As = smem;                 // [2][BM * LDK]
    float *const Bs = smem + 2 * BM * LDK;  // [2][BN * LDK]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN, wn = wave - (wave / WGN) * WGN;

    // XCD-aware tile order: workgroup ids are dealt round-robin to the 8 XCDs, so give XCD x
    // the contiguous logical range [x * per, (x + 1) * per) of the tiles (N fastest).
    const int nb = gridDim.x;
    const int full = nb & ~7;
    int lin = blockIdx.x;
    if (lin < full) {
        const int per = full >> 3;
        lin = (lin & 7) * per + (lin >> 3);
    }
    const int tm = lin / p.tiles_n;
    const int tn = lin - tm * p.tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;

    const int bz = blockIdx.z / p.split;
    const int ks = blockIdx.z - bz * p.split;
    long ao, bo, co, ro;
    batch_offsets(p, bz, ao, bo, co, ro);
    const float *abase = p.a.p + ao;
    const float *bbase = p.b.p + bo;
    const int kbeg = ks * p.kchunk;
    const int kend = min(p.K, kbeg + p.kchunk);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

    // ---- per-thread loader state ----------------------------------------------------------
    // Vector paths: thread t loads rows (t >> 3) + 32 r, k quad (t & 7) * 4 of each stage.
    // Generic paths: thread t loads rows (t >> 5) + 8 r, k = t & 31 of each stage.
    const int kq = (tid & 7) * 4;
    const int kg = tid & 31;
    constexpr int AROWS = AMODE == AM_GEN ? AG : AV;
    const float *arow[AROWS];
    int aih[AROWS], aiw[AROWS];
    {
        const int ohw = p.a.OH * p.a.OW;
#pragma unroll
        for (int r = 0; r < AROWS; ++r) {
            const int m = m0 + (AMODE == AM_GEN ? (tid >> 5) + 8 * r : (tid >> 3) + 32 * r);
            arow[r] = nullptr;
            aih[r] = aiw[r] = 0;
            if (m < p.M) {
                if (p.a.kind == MGC_OP_CONV_NHWC) {
                    int n = m / ohw, rr = m - n * ohw;
                    int oh = rr / p.a.OW, ow = rr - oh * p.a.OW;
                    arow[r] = abase + (long)n * p.a.H * p.a.W * p.a.C;
                    aih[r] = oh * p.a.SH - p.a.PT;
                    aiw[r] = ow * p.a.SW - p.a.PL;
                } else {
                    arow[r] = abase + (long)m * p.a.rs;
                }
            }
        }
    }
    const float *brow[BV];
    if constexpr (BMODE == BD_NK_VEC) {
#pragma unroll
        for (int r = 0; r < BV; ++r) {
            int n = n0 + (tid >> 3) + 32 * r;
            brow[r] = n < p.N ? bbase + (long)n * p.b.cs : nullptr;
        }
    }

    f4 areg[AMODE == AM_GEN ? 1 : AV];
    float agen[AMODE == AM_GEN ? AG : 1];
    f4 breg[BMODE == BD_GEN ? 1 : BV];
    float bgen[BMODE == BD_GEN ? BG : 1];
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const float *const asafe = p.a.p;
    const float *const bsafe = p.b.p;

    auto load_stage = [&](int kt) __attribute__((always_inline)) {
        const int k0 = kbeg + kt * BK;
        if constexpr (AMODE == AM_VEC) {
            const int k = k0 + kq;
            const bool kok = k < kend;
#pragma unroll
            for (int r = 0; r < AV; ++r) {
                const bool ok = kok && arow[r] != nullptr;
                f4 v = *reinterpret_cast<const f4 *>(ok ? arow[r] + k : asafe);
                areg[r] = ok ? v : zero4;
            }
        } else if constexpr (AMODE == AM_CONV_VEC) {
            const int k = k0 + kq;
            const bool kok = k < kend;
            const int t = k / p.a.cg;
            const int c = k - t * p.a.cg;
            const int kh = t / p.a.KW, kw = t - (t / p.a.KW) * p.a.KW;
            const int dh = kh * p.a.DH, dw = kw * p.a.DW;
#pragma unroll
            for (int r = 0; r < AV; ++r) {
                const int ih = aih[r] + dh, iw = aiw[r] + dw;
                const bool ok = kok && arow[r] != nullptr && (unsigned)ih < (unsigned)p.a.H &&
                                (unsigned)iw < (unsigned)p.a.W;
                f4 v = *reinterpret_cast<const f4 *>(
                    ok ? arow[r] + ((long)ih * p.a.W + iw) * p.a.C + c : asafe);
                areg[r] = ok ? v : zero4;
            }
        } else {
            const int k = k0 + kg;
            const bool kok = k < kend;
            if (p.a.kind == MGC_OP_CONV_NHWC) {
                const int t = k / p.a.cg;
                const int c = k - t * p.a.cg;
                const int kh = t / p.a.KW, kw = t - (t / p.a.KW) * p.a.KW;
                const int dh = kh * p.a.DH, dw = kw * p.a.DW;
#pragma unroll
                for (int r = 0; r < AG; ++r) {
                    const int ih = aih[r] + dh, iw = aiw[r] + dw;
                    const bool ok = kok && arow[r] != nullptr && (unsigned)ih < (unsigned)p.a.H &&
                                    (unsigned)iw < (unsigned)p.a.W;
                    float v = *(ok ? arow[r] + ((long)ih * p.a.W + iw) * p.a.C + c : asafe);
                    agen[r] = ok ? v : 0.0f;
                }
            } else {
#pragma unroll
                for (int r = 0; r < AG; ++r) {
                    const bool ok = kok && arow[r] != nullptr;
                    float v = *(ok ? arow[r] + (long)k * p.a.cs : asafe);
                    agen[r] = ok ? v : 0.0f;
                }
            }
        }
        if constexpr (BMODE == BD_NK_VEC) {
            const int k = k0 + kq;
            const bool kok = k < kend;
#pragma unroll
            for (int r = 0; r < BV; ++r) {
                const bool ok = kok && brow[r] != nullptr;
                f4 v = *reinterpret_cast<const f4 *>(ok ? brow[r] + k : bsafe);
                breg[r] = ok ? v : zero4;
            }
        } else if constexpr (BMODE == BD_KN_VEC) {
#pragma unroll
            for (int r = 0; r < BV; ++r) {
                const int e = tid + 256 * r;
                const int krow = e / (BN / 4);
                const int nq = (e - krow * (BN / 4)) * 4;
                const int k = k0 + krow, n = n0 + nq;
                const bool ok = k < kend && n < p.N;
                f4 v = *reinterpret_cast<const f4 *>(ok ? bbase + (long)k * p.b.rs + n : bsafe);
                breg[r] = ok ? v : zero4;
            }
        } else {
            const int k = k0 + kg;
            const bool kok = k < kend;
            if (p.b.kind == MGC_OP_CONV_NCHW) {
                const mgc_hip_operand &o = p.b;
                const int t = k / o.KW, kw = k - (k / o.KW) * o.KW;
                const int c = t / o.KH, kh = t - (t / o.KH) * o.KH;
                const float *plane = bbase + (long)c * o.H * o.W;
#pragma unroll
                for (int r = 0; r < BG; ++r) {
                    const int n = n0 + (tid >> 5) + 8 * r;
                    const int oh = n / o.OW, ow = n - (n / o.OW) * o.OW;
                    const int ih = oh * o.SH - o.PT + kh * o.DH, iw = ow * o.SW - o.PL + kw * o.DW;
                    const bool ok = kok && n < p.N && (unsigned)ih < (unsigned)o.H &&
                                    (unsigned)iw < (unsigned)o.W;
                    float v = *(ok ? plane + (long)ih * o.W + iw : bsafe);
                    bgen[r] = ok ? v : 0.0f;
                }
            } else {
#pragma unroll
                for (int r = 0; r < BG; ++r) {
                    const int n = n0 + (tid >> 5) + 8 * r;
                    const bool ok = kok && n < p.N;
                    float v = *(ok ? bbase + (long)k * p.b.rs + (long)n * p.b.cs : bsafe);
                    bgen[r] = ok ? v : 0.0f;
                }
            }
        }
    };

    auto store_stage = [&](int buf) __attribute__((always_inline)) {
        float *as = As + buf * BM * LDK;
        float *bs = Bs + buf * BN * LDK;
        if constexpr (AMODE == AM_GEN) {
#pragma unroll
            for (int r = 0; r < AG; ++r) as[((tid >> 5) + 8 * r) * LDK + kg] = agen[r];
        } else {
#pragma unroll
            for (int r = 0; r < AV; ++r)
                *reinterpret_cast<f4 *>(&as[((tid >> 3) + 32 * r) * LDK + kq]) = areg[r];
        }
        if constexpr (BMODE == BD_GEN) {
#pragma unroll
            for (int r = 0; r < BG; ++r) bs[((tid >> 5) + 8 * r) * LDK + kg] = bgen[r];
        } else if constexpr (BMODE == BD_KN_VEC) {
#pragma unroll
            for (int r = 0; r < BV; ++r) {
                const int e = tid + 256 * r;
                const int krow = e / (BN / 4);
                const int nq = (e - krow * (BN / 4)) * 4;
                bs[(nq + 0) * LDK + krow] = breg[r][0];
                bs[(nq + 1) * LDK + krow] = breg[r][1];
                bs[(nq + 2) * LDK + krow] = breg[r][2];
                bs[(nq + 3) * LDK + krow] = breg[r][3];
            }
        } else {
#pragma unroll
            for (int r = 0; r < BV; ++r)
                *reinterpret_cast<f4 *>(&bs[((tid >> 3) + 32 * r) * LDK + kq]) = breg[r];
        }
    };

    floatx16 acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int li = lane & 31;
    const int lh = lane >> 5;

    if (nk > 0) {
        load_stage(0);
        store_stage(0);
        __syncthreads();
    }
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_stage(kt + 1);
        const float *as = As + buf * BM * LDK;
        const float *bs = Bs + buf * BN * LDK;
        f4 af[RM][4], bf[RN][4];
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                af[i][s] = *reinterpret_cast<const f4 *>(
                    &as[(wm * WM + i * 32 + li) * LDK + lh * 16 + 4 * s]);
#pragma unroll
        for (int j = 0; j < RN; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                bf[j][s] = *reinterpret_cast<const f4 *>(
                    &bs[(wn * WN + j * 32 + li) * LDK + lh * 16 + 4 * s]);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < RM; ++i)
#pragma unroll
                    for (int j = 0; j < RN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s][e], bf[j][s][e],
                                                                          acc[i][j], 0, 0, 0);
        if (kt + 1 < nk) store_stage(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue, pass 1: registers -> LDS tile. Block (i, j) register r holds tile row
    // 8 * (r / 4) + 4 * lh + r % 4 and column li of that 32x32 block.
    float *const Cs = smem;
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                Cs[(wm * WM + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3)) * LDC + wn * WN + j * 32 +
                   li] = acc[i][j][r];
    __syncthreads();

    // ---- epilogue, pass 2: 16-byte chunks of the tile, compact loop ------------------------
    constexpr int C4 = BN / 4;
    const bool split_out = p.split > 1;
    float *const cbase = split_out ? p.ws + (long)ks * p.M * p.N : p.c + co;
    const long ldc = split_out ? (long)p.N : p.ldc;
    const float *const rbase = (!split_out && p.res) ? p.res + ro : nullptr;
    const bool vec = split_out ? (p.N % 4 == 0) : (p.vec_out != 0);
#pragma unroll 1
    for (int idx = tid; idx < BM * C4; idx += 256) {
        const int rl = idx / C4;
        const int cl = (idx - rl * C4) * 4;
        const int row = m0 + rl, col = n0 + cl;
        if (row >= p.M || col >= p.N) continue;
        f4 v = *reinterpret_cast<const f4 *>(&Cs[rl * LDC + cl]);
        const int ncol = min(4, p.N - col);
        float *dst = cbase + (long)row * ldc + col;
        if (split_out) {
            if (vec && ncol == 4) {
                *reinterpret_cast<f4 *>(dst) = v;
            } else {
                for (int e = 0; e < ncol; ++e) dst[e] = v[e];
            }
            continue;
        }
        v *= p.alpha;
        if (p.bias) {
            if (p.bias_mode == 2) {
                v += p.bias[row];
            } else if (vec && ncol == 4) {
                v += *reinterpret_cast<const f4 *>(p.bias + col);
            } else {
                for (int e = 0; e < ncol; ++e) v[e] += p.bias[col + e];
            }
        }
        if (rbase) {
            const float *src = rbase + (long)row * p.ldr + col;
            if (vec && ncol == 4) {
                v += p.beta * *reinterpret_cast<const f4 *>(src);
            } else {
                for (int e = 0; e < ncol; ++e) v[e] += p.beta * src[e];
            }
        }
        v = act4(v, p.act, p.lo, p.hi);
        if (vec && ncol == 4) {
            *reinterpret_cast<f4 *>(dst) = v;
        } else {
            for (int e = 0; e < ncol; ++e) dst[e] = v[e];
        }
    }
}

// Sum the split-K partials and apply the epilogue (one batch element).
__global__ void gemm_splitk_reduce(const GemmDev p) {
    const long total = (long)p.M * p.N;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        const int row = (int)(idx / p.N), col = (int)(idx - (long)(idx / p.N) * p.N);
        float v = 0.0f;
        for (int s = 0; s < p.split; ++s) v += p.ws[(long)s * total + idx];
        v = p.alpha * v;
        if (p.bias && p.bias_mode == 2) v += p.bias[row];
        if (p.bias && p.bias_mode == 1) v += p.bias[col];
        if (p.res) v += p.beta * p.res[(long)row * p.ldr + col];
        p.c[(long)row * p.ldc + col] = apply_act(v, p.act, p.lo, p.hi);
    }
}

static bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15) == 0; }

static bool bs_div4(const long *bs, int rank) {
    for (int d = 0; d < rank; ++d)
        if (bs[d] % 4) return false;
    return true;
}

typedef void (*GemmKernel)(const GemmDev);

template <int BM, int BN, int WGM>
static GemmKernel pick_kernel(int am, int bm) {
#define MGC_K(A, B) &gemm_mfma_kernel<BM, BN, WGM, A, B>
    static const GemmKernel table[3][3] = {
        {MGC_K(AM_VEC, BD_NK_VEC), MGC_K(AM_VEC, BD_KN_VEC), MGC_K(AM_VEC, BD_GEN)},
        {MGC_K(AM_CONV_VEC, BD_NK_VEC), MGC_K(AM_CONV_VEC, BD_KN_VEC), MGC_K(AM_CONV_VEC, BD_GEN)},
        {MGC_K(AM_GEN, BD_NK_VEC), MGC_K(AM_GEN, BD_KN_VEC), MGC_K(AM_GEN, BD_GEN)},
    };
#undef MGC_K
    return table[am][bm];
}

struct TileChoice {
    int bm, bn, split;
};

static const int kCUs = 256;

// Tile shape and K split for one GEMM. Larger tiles reuse more data per LDS stage; the chip
// needs several hundred workgroups in flight, so small problems drop to 64-wide tiles and,
// failing that, split K.
static TileChoice choose_tiles(int M, int N, int K, int batch) {
    TileChoice t;
    t.bn = N <= 64 ? 64 : 128;
    t.bm = 128;
    long tiles = (long)((M + 127) / 128) * ((N + t.bn - 1) / t.bn) * batch;
    if (tiles < 2 * kCUs) {
        t.bm = 64;
        t.bn = 64;
    }
    tiles = (long)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
    t.split = 1;
    if (batch == 1 && tiles < kCUs && K >= 512) {
        int want = (int)((2 * kCUs + tiles - 1) / tiles);
        int max_split = K / 256;
        t.split = want < max_split ? want : max_split;
        if (t.split < 1) t.split = 1;
    }
    return t;
}

}  // namespace mgc

using namespace mgc;

extern "C" long mgc_hip_gemm_workspace(int M, int N, int K, int batch) {
    TileChoice t = choose_tiles(M, N, K, batch);
    return t.split > 1 ? (long)t.split * M * N : 0;
}

extern "C" void mgc_hip_gemm(mgc_hip_exec *x, const mgc_hip_gemm_args *g) {
    if (g->M <= 0 || g->N <= 0) return;
    GemmDev p;
    p.M = g->M;
    p.N = g->N;
    p.K = g->K;
    p.a = g->a;
    p.b = g->b;
    p.c = g->c;
    p.ldc = g->ldc;
    p.alpha = g->alpha;
    p.beta = g->beta;
    p.bias = g->bias;
    p.bias_mode = g->bias ? g->bias_mode : 0;
    p.res = g->res;
    p.ldr = g->ldr;
    p.act = g->act;
    p.lo = g->lo;
    p.hi = g->hi;
    p.batch_rank = g->batch_rank;
    int batch = 1;
    for (int d = 0; d < 4; ++d) {
        p.bdims[d] = d < g->batch_rank ? g->batch_dims[d] : 1;
        p.a_bs[d] = d < g->batch_rank ? g->a_bs[d] : 0;
        p.b_bs[d] = d < g->batch_rank ? g->b_bs[d] : 0;
        p.c_bs[d] = d < g->batch_rank ? g->c_bs[d] : 0;
        p.r_bs[d] = d < g->batch_rank ? g->r_bs[d] : 0;
        if (d < g->batch_rank) batch *= g->batch_dims[d];
    }
    if (batch <= 0) return;

    int am = AM_GEN;
    if (p.a.kind == MGC_OP_STRIDED && p.a.cs == 1 && p.a.rs % 4 == 0 && p.K % 4 == 0 &&
        aligned16(p.a.p) && bs_div4(p.a_bs, p.batch_rank))
        am = AM_VEC;
    else if (p.a.kind == MGC_OP_CONV_NHWC && p.a.cg % 4 == 0 && p.a.C % 4 == 0 &&
             aligned16(p.a.p) && bs_div4(p.a_bs, p.batch_rank))
        am = AM_CONV_VEC;
    int bm = BD_GEN;
    if (p.b.kind == MGC_OP_STRIDED && p.b.rs == 1 && p.b.cs % 4 == 0 && p.K % 4 == 0 &&
        aligned16(p.b.p) && bs_div4(p.b_bs, p.batch_rank))
        bm = BD_NK_VEC;
    else if (p.b.kind == MGC_OP_STRIDED && p.b.cs == 1 && p.b.rs % 4 == 0 && p.N % 4 == 0 &&
             aligned16(p.b.p) && bs_div4(p.b_bs, p.batch_rank))
        bm = BD_KN_VEC;

    p.vec_out = p.ldc % 4 == 0 && aligned16(p.c) && bs_div4(p.c_bs, p.batch_rank) &&
                (!p.res || (p.ldr % 4 == 0 && aligned16(p.res) && bs_div4(p.r_bs, p.batch_rank))) &&
                (!p.bias || p.bias_mode != 1 || aligned16(p.bias));

    TileChoice t = choose_tiles(p.M, p.N, p.K, batch);
    if (t.split > 1 && (g->workspace == nullptr ||
                        g->workspace_floats < (long)t.split * p.M * p.N)) {
        t.split = 1;
    }
    if (g->split_k > 0 && batch == 1) {
        t.split = g->split_k;
        if (t.split > 1 && (g->workspace == nullptr ||
                            g->workspace_floats < (long)t.split * p.M * p.N))
            t.split = 1;
    }
    p.split = t.split;
    int kchunk = (p.K + t.split - 1) / t.split;
    p.kchunk = (kchunk + 31) / 32 * 32;
    if (p.kchunk == 0) p.kchunk = 32;
    p.ws = g->workspace;
    p.tiles_m = (p.M + t.bm - 1) / t.bm;
    p.tiles_n = (p.N + t.bn - 1) / t.bn;

    GemmKernel kern;
    if (t.bm == 128 && t.bn == 128)
        kern = pick_kernel<128, 128, 2>(am, bm);
    else if (t.bm == 128 && t.bn == 64)
        kern = pick_kernel<128, 64, 2>(am, bm);
    else
        kern = pick_kernel<64, 64, 2>(am, bm);

    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)(batch * p.split));
    MGC_LAUNCH(x, kern, grid, dim3(256), 0, p);
    if (p.split > 1) {
        MGC_LAUNCH(x, gemm_splitk_reduce, dim3(blocks_for((long)p.M * p.N, 256, 4096)), dim3(256),
                   0, p);
    }
}
