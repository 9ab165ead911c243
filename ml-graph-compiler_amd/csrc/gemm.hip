// fp32 GEMM and implicit-GEMM convolution on CDNA4 matrix cores (v_mfma_f32_32x32x2f32).
//
// Computes C[z] = act(alpha * A[z] B[z] + bias + beta * R[z]), the contract of the reference's
// mgc_gemm (src/ml_graph_compiler/codegen/runtime/mgc_kernels.c:282-396), with operands read as
// strided matrices or through implicit im2col of an NHWC (A) or NCHW (B) image.
//
// Two kernels share the MFMA core (MI355X-first, not a translation of the reference's
// Goto/BLIS CPU blocking). A workgroup of 256 threads (4 waves of 64) owns a BM x BN output
// tile; each wave owns a WM x WN sub-tile of 32x32 MFMA blocks (16 accumulators per block).
// K advances 32 per stage; the 32x32x2 MFMA consumes two k per instruction, one per half-wave,
// and the kernels give the first 16 k of a stage to lanes 0-31 and the last 16 to lanes 32-63
// (a permutation of the summation order applied identically to A and B), so a lane's
// operands are contiguous 16-byte LDS reads.
//
//  * gemm_dma_kernel (k-contiguous operands: packed weights, NHWC activations, row-major
//    matrices — every convolution and linear layer). Tiles travel from HBM to LDS with
//    buffer_load_dwordx4 ... lds (no register staging) through a ring of stages; masked
//    elements use an offset past the end of the buffer resource, which the hardware reads as
//    zero. The LDS row layout is fixed by the DMA (a wave's 64 lanes write 1 KB of consecutive
//    LDS), so bank spreading comes from which k-chunk each lane fetches (an XOR swizzle).
//    Barriers wait only for LDS traffic, so the loads of later stages stay in flight.
//    Implicit-im2col offsets are advanced incrementally and divisions by shape constants use
//    host-computed magic numbers.
//  * gemm_mfma_kernel: every other operand form (transposed or strided A, NCHW im2col B,
//    dynamic k-major B), staged through registers into double-buffered LDS.
//  * The workgroup id is remapped so each of the 8 XCDs (each with its own L2) works on a
//    contiguous range of tiles, N fastest: tiles that share A rows share an L2.
//  * Tiles are 64 x 64 (see choose_tiles); K is split over extra workgroups into a
//    planner-provided workspace when the tiles alone cannot balance the CUs, and a reduction
//    then applies the epilogue.
#include <stdio.h>

#include <mutex>

#include "mgc_device.h"

namespace mgc {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned uint4_t __attribute__((ext_vector_type(4)));

// A operand forms: strided with unit column stride, NHWC image (implicit im2col), generic
// (register-staged), and a concatenation of a strided matrix (columns < k1) with an NHWC image
// read as a strided 1 x 1 convolution (columns >= k1).
enum { AM_VEC = 0, AM_CONV_VEC = 1, AM_GEN = 2, AM_CAT = 3 };

// 16 zero bytes: the load address of every out-of-range operand element.
__device__ __attribute__((aligned(16))) float g_zero_page[4] = {0.0f, 0.0f, 0.0f, 0.0f};

// Loads through the global address space. Every operand lives in device memory; saying so
// keeps the compiler from falling back to flat loads, which share a wait counter with LDS.
typedef const __attribute__((address_space(1))) float gfloat;
typedef const __attribute__((address_space(1))) f4 gf4;
__device__ __forceinline__ float ldg(const float *ptr) { return *(gfloat *)ptr; }
__device__ __forceinline__ f4 ldg4(const float *ptr) { return *(gf4 *)ptr; }
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
    int vec_out;
    FastDiv div_ow, div_ohw, div_cg, div_kw;  // A as NHWC image: OW, OH * OW, cg, KW
    long a_bytes, b_bytes;  // bytes of A and B reachable from a.p / b.p (all batch elements)
    mgc_hip_operand a2;     // AM_CAT: the image whose 1 x 1 strided window gives columns >= k1
    int k1;
    long a2_bytes;
    int nbatch;   // batch elements
    int nfull = 0x7fffffff;  // gemm_dma_kernel: workgroups from this id on compute quarter tiles
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

// Epilogue shared by the GEMM kernels, pass 2: the BM x BN tile, staged in LDS at Cs with row
// pitch BN + 8 floats, leaves as 16-byte chunks with alpha, bias, residual and activation
// applied, or raw into the split-K workspace. Each thread owns one fixed 16-byte column chunk
// of the tile and the rows r0, r0 + RSTEP, ..., so the column bias is read once per thread.
// Every one of the 256 threads calls it (no barrier inside).
template <int BM, int BN>
__device__ __forceinline__ void gemm_lds_to_global(const GemmDev &p, const float *Cs, int m0, int n0, int ks,
                                                   long co, long ro) {
    constexpr int LDC = BN + 8;
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const int tid = threadIdx.x;
    constexpr int C4 = BN / 4;
    static_assert(256 % C4 == 0, "column chunks must divide the workgroup");
    constexpr int RSTEP = 256 / C4;
    constexpr int ITERS = BM / RSTEP;
    constexpr int G = ITERS < 4 ? ITERS : 4;
    // Scalars read once: keeps the compiler from copying the argument block to scratch.
    const float alpha = p.alpha, beta = p.beta, lo = p.lo, hi = p.hi;
    const float *const bias = p.bias;
    const int act = p.act, M = p.M, N = p.N;
    const bool split_out = p.split > 1;
    float *const cbase = split_out ? p.ws + (long)ks * M * N : p.c + co;
    const long ldc = split_out ? (long)N : p.ldc;
    const float *const rbase = (!split_out && p.res) ? p.res + ro : nullptr;
    const bool vec = split_out ? (N % 4 == 0) : (p.vec_out != 0);
    const int cl = (tid % C4) * 4;
    const int col = n0 + cl;
    const int r0 = tid / C4;
    const bool col_ok = col < N;
    const int ncol = col_ok ? min(4, N - col) : 0;
    const bool full4 = vec && ncol == 4;
    const int bmode = split_out ? 0 : p.bias_mode;
    f4 cbias = zero4;
    if (bmode == 1 && col_ok) {
        if (full4) {
            cbias = ldg4(bias + col);
        } else {
            for (int e = 0; e < ncol; ++e) cbias[e] = ldg(bias + col + e);
        }
    }
    // pass 2: LDS tile -> epilogue -> memory, 16 bytes per access, G rows per step with their
    // residual chunks (and row biases) requested together.
    if (!col_ok) return;
    const bool pre_res = rbase != nullptr && full4;
#pragma unroll 1
    for (int g = 0; g < ITERS; g += G) {
        f4 rv[G];
        float rb[G];
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const int row = m0 + r0 + RSTEP * (g + u);
            const bool ok = row < M;
            rv[u] = zero4;
            rb[u] = 0.0f;
            if (pre_res)
                rv[u] = ldg4(ok ? rbase + (long)row * p.ldr + col
                                                         : g_zero_page);
            if (bmode == 2) rb[u] = ldg(ok ? bias + row : g_zero_page);
        }
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const int rl = r0 + RSTEP * (g + u);
            const int row = m0 + rl;
            if (row >= M) break;
            f4 v = *reinterpret_cast<const f4 *>(&Cs[rl * LDC + cl]);
            float *dst = cbase + (long)row * ldc + col;
            if (!split_out) {
                v = v * alpha + cbias;
                if (bmode == 2) v += rb[u];
                if (pre_res) {
                    v += beta * rv[u];
                } else if (rbase) {
                    const float *src = rbase + (long)row * p.ldr + col;
                    for (int e = 0; e < ncol; ++e) v[e] += beta * ldg(src + e);
                }
                v = act4(v, act, lo, hi);
            }
            if (full4) {
                *reinterpret_cast<f4 *>(dst) = v;
            } else {
                for (int e = 0; e < ncol; ++e) dst[e] = v[e];
            }
        }
    }
}




// The whole epilogue: pass 1 moves the accumulators to LDS (smem, at least BM * (BN + 8)
// floats, free when this is called), then gemm_lds_to_global.
template <int BM, int BN, int WGM, int RM, int RN>
__device__ __forceinline__ void gemm_store_tile(const GemmDev &p, float *smem,
                                                     const floatx16 (&acc)[RM][RN], int m0, int n0,
                                                     int ks, long co, long ro) {
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM;
    constexpr int WN = BN / WGN;
    constexpr int LDC = BN + 8;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN, wn = wave - (wave / WGN) * WGN;
    const int li = lane & 31;
    const int lh = lane >> 5;
    // pass 1: registers -> LDS tile. Block (i, j) register r holds tile row
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
    gemm_lds_to_global<BM, BN>(p, Cs, m0, n0, ks, co, ro);
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
    constexpr int LDC = BN + 8;
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
    // Out-of-range elements load from a zero page instead of being masked after the load: a
    // select on the loaded value would make the wave wait for the load right where it is
    // issued instead of where the value is consumed, one pipeline stage later.
    const float *const asafe = g_zero_page;
    const float *const bsafe = g_zero_page;

    auto load_stage = [&](int kt) __attribute__((always_inline)) {
        const int k0 = kbeg + kt * BK;
        if constexpr (AMODE == AM_VEC) {
            const int k = k0 + kq;
            const bool kok = k < kend;
#pragma unroll
            for (int r = 0; r < AV; ++r) {
                const bool ok = kok && arow[r] != nullptr;
                areg[r] = ldg4(ok ? arow[r] + k : asafe);
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
                areg[r] = ldg4(ok ? arow[r] + ((long)ih * p.a.W + iw) * p.a.C + c : asafe);
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
                    agen[r] = ldg(ok ? arow[r] + ((long)ih * p.a.W + iw) * p.a.C + c : asafe);
                }
            } else {
#pragma unroll
                for (int r = 0; r < AG; ++r) {
                    const bool ok = kok && arow[r] != nullptr;
                    agen[r] = ldg(ok ? arow[r] + (long)k * p.a.cs : asafe);
                }
            }
        }
        if constexpr (BMODE == BD_NK_VEC) {
            const int k = k0 + kq;
            const bool kok = k < kend;
#pragma unroll
            for (int r = 0; r < BV; ++r) {
                const bool ok = kok && brow[r] != nullptr;
                breg[r] = ldg4(ok ? brow[r] + k : bsafe);
            }
        } else if constexpr (BMODE == BD_KN_VEC) {
#pragma unroll
            for (int r = 0; r < BV; ++r) {
                const int e = tid + 256 * r;
                const int krow = e / (BN / 4);
                const int nq = (e - krow * (BN / 4)) * 4;
                const int k = k0 + krow, n = n0 + nq;
                const bool ok = k < kend && n < p.N;
                breg[r] = ldg4(ok ? bbase + (long)k * p.b.rs + n : bsafe);
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
                    bgen[r] = ldg(ok ? plane + (long)ih * o.W + iw : bsafe);
                }
            } else {
#pragma unroll
                for (int r = 0; r < BG; ++r) {
                    const int n = n0 + (tid >> 5) + 8 * r;
                    const bool ok = kok && n < p.N;
                    bgen[r] = ldg(ok ? bbase + (long)k * p.b.rs + (long)n * p.b.cs : bsafe);
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

    gemm_store_tile<BM, BN, WGM>(p, smem, acc, m0, n0, ks, co, ro);
}

// s_waitcnt with only the vector-memory counter constrained (expcnt and lgkmcnt at maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// Workgroup barrier for the LDS ring: waits for this wave's own LDS accesses only. The
// __syncthreads() fence would also wait for every outstanding global load, including the
// DMA loads of later pipeline stages, and drain the ring at every step.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes at byte offset voff of a buffer resource straight into LDS (lane l of the wave
// writes lds_base + 16 * l); offsets at or past the resource's size read as zeros.
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, unsigned voff, float *lds_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_base, 16, (int)voff, 0, 0, 0);
}


// GEMM / implicit-GEMM convolution for k-contiguous operands (A: strided with unit column
// stride, or an NHWC image with channel groups divisible by 4; B: packed [N][K]).
//  * Operand tiles travel global -> LDS with global_load_lds_dwordx4 (no register staging)
//    through a STAGES-deep ring, so loads for stage kt + STAGES - 1 are in flight while stage kt
//    is multiplied; one barrier per stage.
//  * Each stage stores a BM x 32 (and BN x 32) float block as rows of eight 16-byte chunks.
//    The DMA writes a wave's 64 lanes to 1 KB of consecutive LDS, so the row layout is fixed
//    by the lane order; the bank spread comes from which chunk a lane fetches: lane l loads
//    k-chunk (l & 7) ^ (l >> 3) of row l >> 3 of its 8-row group, i.e. LDS position p of row r
//    holds k-chunk p ^ (r & 7). The fragment reads undo that XOR, and eight lanes reading the
//    same k-chunk of eight consecutive rows hit eight different positions.
template <int BM, int BN, int WGM, int STAGES, int AMODE>
__global__ void __launch_bounds__(256) gemm_dma_kernel(const GemmDev p) {
    constexpr int BK = 32;
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM;
    constexpr int WN = BN / WGN;
    constexpr int RM = WM / 32;
    constexpr int RN = WN / 32;
    static_assert(RM >= 1 && RN >= 1 && WGM * WGN == 4, "bad tile");
    static_assert(STAGES >= 2 && STAGES <= 4, "stages");
    constexpr int AI = BM / 32;  // DMA instructions per wave per stage, A block
    constexpr int BI = BN / 32;  // and B block
    constexpr int STAGE = (BM + BN) * BK;
    constexpr int SMEM_LOOP = STAGES * STAGE;
    constexpr int SMEM_EPI = BM * (BN + 8);
    constexpr int SMEM = SMEM_LOOP > SMEM_EPI ? SMEM_LOOP : SMEM_EPI;
    static_assert(AMODE == AM_VEC || AMODE == AM_CONV_VEC || AMODE == AM_CAT, "vector A only");

    __shared__ __attribute__((aligned(16))) float smem[SMEM];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave - (wave / WGN) * WGN;

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

    // ---- DMA source state: row (i * 4 + wave) * 8 + (lane >> 3) of each block --------------
    // Row r keeps k-chunk q at position q ^ f(r) with f(r) = (r & 7) ^ ((r >> 3) & 1): distinct
    // over any 8 consecutive rows and over the 8 even (or odd) rows of any aligned 16, so
    // 16-byte reads of one chunk from 8 or 16 consecutive rows spread over all banks.
    const int q4 = ((lane & 7) ^ (lane >> 3) ^ (wave & 1)) * 4;  // this lane's k offset
    const int rsub = lane >> 3;
    // Operands are read through buffer resources: a masked lane gets an offset past the end of
    // the resource and the hardware returns zeros for it, so no zero page, no select after
    // the load and 32-bit offsets instead of 64-bit addresses.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)abase, (short)0, (int)(p.a_bytes - ao * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)bbase, (short)0, (int)(p.b_bytes - bo * 4), 0x00020000);
    constexpr unsigned OOB = 0x80000000u;  // past every resource's end (extents are < 2^31 bytes)
    // AM_CAT: the second source (batch_rank 0, so no batch offset)
    const __amdgpu_buffer_rsrc_t ra2 = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(AMODE == AM_CAT ? p.a2.p : abase), (short)0, (int)(AMODE == AM_CAT ? p.a2_bytes : 0), 0x00020000);
    unsigned aoff[AI];  // byte offset of the row (AM_VEC) or of its window origin (AM_CONV_VEC)
    unsigned aoff2[AI];  // AM_CAT: byte offset of the row's pixel in the second source
    int aih[AI], aiw[AI];
    const int ohw = AMODE == AM_CAT ? p.a2.OH * p.a2.OW : p.a.OH * p.a.OW;
#pragma unroll
    for (int i = 0; i < AI; ++i) {
        const int m = m0 + (i * 4 + wave) * 8 + rsub;
        aoff[i] = aoff2[i] = OOB;
        aih[i] = aiw[i] = -0x40000000;  // fails the window bounds test
        if (m < p.M) {
            if (AMODE == AM_CAT) {
                const int n = fdiv(m, p.div_ohw), rr = m - n * ohw;
                const int oh = fdiv(rr, p.div_ow), ow = rr - oh * p.a2.OW;
                aoff2[i] = (unsigned)(((n * p.a2.H + oh * p.a2.SH) * p.a2.W + ow * p.a2.SW) * p.a2.C) * 4u;
            }
            if (AMODE == AM_CONV_VEC) {
                const int n = fdiv(m, p.div_ohw), rr = m - n * ohw;
                const int oh = fdiv(rr, p.div_ow), ow = rr - oh * p.a.OW;
                aih[i] = oh * p.a.SH - p.a.PT;
                aiw[i] = ow * p.a.SW - p.a.PL;
                aoff[i] = (unsigned)(((n * p.a.H + aih[i]) * p.a.W + aiw[i]) * p.a.C) * 4u;
            } else {
                aoff[i] = (unsigned)m * (unsigned)p.a.rs * 4u;
            }
        }
    }
    unsigned boff[BI];
#pragma unroll
    for (int i = 0; i < BI; ++i) {
        const int n = n0 + (i * 4 + wave) * 8 + rsub;
        boff[i] = n < p.N ? (unsigned)n * (unsigned)p.b.cs * 4u : OOB;
    }
    // The lane's next k and, for an image, its (kh, kw, c) split, advanced one stage per issue.
    int knext = kbeg + q4;
    int cc = 0, ckw = 0, ckh = 0;
    if (AMODE == AM_CONV_VEC) {
        const int t = fdiv(knext, p.div_cg);
        cc = knext - t * p.a.cg;
        ckh = fdiv(t, p.div_kw);
        ckw = t - ckh * p.a.KW;
    }

    auto issue = [&](int buf) __attribute__((always_inline)) {
        const int k = knext;
        const bool kok = k < kend;
        float *sa = smem + buf * STAGE;
        float *sb = sa + BM * BK;
        if constexpr (AMODE == AM_VEC) {
#pragma unroll
            for (int i = 0; i < AI; ++i)
                dma16_buf(ra, kok ? aoff[i] + (unsigned)k * 4u : OOB, sa + (i * 4 + wave) * 8 * BK);
        } else if constexpr (AMODE == AM_CAT) {
            // k1 is a multiple of the 32-wide stage, so a whole stage reads one source
            if (k < p.k1) {
#pragma unroll
                for (int i = 0; i < AI; ++i)
                    dma16_buf(ra, kok ? aoff[i] + (unsigned)k * 4u : OOB, sa + (i * 4 + wave) * 8 * BK);
            } else {
                const unsigned k2 = (unsigned)(k - p.k1) * 4u;
#pragma unroll
                for (int i = 0; i < AI; ++i)
                    dma16_buf(ra2, kok ? aoff2[i] + k2 : OOB, sa + (i * 4 + wave) * 8 * BK);
            }
        } else {
            const int dh = ckh * p.a.DH, dw = ckw * p.a.DW;
            const unsigned koff = (unsigned)((dh * p.a.W + dw) * p.a.C + cc) * 4u;
#pragma unroll
            for (int i = 0; i < AI; ++i) {
                const bool ok = kok && (unsigned)(aih[i] + dh) < (unsigned)p.a.H &&
                                (unsigned)(aiw[i] + dw) < (unsigned)p.a.W;
                dma16_buf(ra, ok ? aoff[i] + koff : OOB, sa + (i * 4 + wave) * 8 * BK);
            }
            cc += BK;
            while (cc >= p.a.cg) {
                cc -= p.a.cg;
                if (++ckw == p.a.KW) {
                    ckw = 0;
                    ++ckh;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < BI; ++i)
            dma16_buf(rb, kok ? boff[i] + (unsigned)k * 4u : OOB, sb + (i * 4 + wave) * 8 * BK);
        knext = k + BK;
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
    const int sw = (li & 7) ^ ((li >> 3) & 1);  // f(row): fragment rows start at multiples of 32

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nk) issue(s);

    constexpr int PER_STAGE = AI + BI;
    for (int kt = 0; kt < nk; ++kt) {
        // Stage kt has landed once at most the later stages' loads are outstanding.
        const int ahead = min(nk - 1 - kt, STAGES - 2);
        if (STAGES >= 4 && ahead >= 2) {
            wait_vmcnt<(STAGES >= 4 ? 2 : 0) * PER_STAGE>();
        } else if (STAGES >= 3 && ahead >= 1) {
            wait_vmcnt<PER_STAGE>();
        } else {
            wait_vmcnt<0>();
        }
        barrier_lds();
        if (kt + STAGES - 1 < nk) issue((kt + STAGES - 1) % STAGES);
        const float *as = smem + (kt % STAGES) * STAGE;
        const float *bs = as + BM * BK;
        f4 af[RM][4], bf[RN][4];
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                af[i][s] = *reinterpret_cast<const f4 *>(
                    &as[(wm * WM + i * 32 + li) * BK + (((lh * 4 + s) ^ sw) << 2)]);
#pragma unroll
        for (int j = 0; j < RN; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                bf[j][s] = *reinterpret_cast<const f4 *>(
                    &bs[(wn * WN + j * 32 + li) * BK + (((lh * 4 + s) ^ sw) << 2)]);
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
    }
    __syncthreads();
    gemm_store_tile<BM, BN, WGM>(p, smem, acc, m0, n0, ks, co, ro);
}

// Body of gemm_dma_tail_kernel: gemm_dma_kernel's whole 64 x 64 tiles, and (QUARTER) a 64 x 64
// tile's 32 x 32 quarter computed by all four waves, each over a quarter of K. A quarter's ring
// stage holds 64 k of its 32 A rows and 32 B rows (LDS row r < 32: k block 0, r >= 32: k block
// 1, same 32-float row format and swizzle), the same 16 KB as a 64 x 64 stage; wave w multiplies the 16 k (w & 1) of k block w >> 1. The
// four partial tiles are summed through LDS in wave order before the common epilogue.
template <int BM, int BN, int STAGES>
constexpr int dma_smem_floats() {
    return STAGES * (BM + BN) * 32 > BM * (BN + 8) ? STAGES * (BM + BN) * 32 : BM * (BN + 8);
}

template <int BM, int BN, int WGM, int STAGES, int AMODE, bool QUARTER>
__device__ __forceinline__ void gemm_dma_tile(const GemmDev p, float *smem, const int m0, const int n0) {
    constexpr int BK = 32;
    constexpr int KSTEP = QUARTER ? 2 * BK : BK;  // k covered by one ring stage
    static_assert(!QUARTER || (BM == 64 && BN == 64 && WGM == 2), "quarters of a 64 x 64 tile");
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM;
    constexpr int WN = BN / WGN;
    constexpr int RM = WM / 32;
    constexpr int RN = WN / 32;
    static_assert(RM >= 1 && RN >= 1 && WGM * WGN == 4, "bad tile");
    static_assert(STAGES >= 2 && STAGES <= 4, "stages");
    constexpr int AI = BM / 32;  // DMA instructions per wave per stage, A block
    constexpr int BI = BN / 32;  // and B block
    constexpr int STAGE = (BM + BN) * BK;
    static_assert(AMODE == AM_VEC || AMODE == AM_CONV_VEC || AMODE == AM_CAT, "vector A only");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave - (wave / WGN) * WGN;

    const int bz = blockIdx.z / p.split;
    const int ks = blockIdx.z - bz * p.split;
    long ao, bo, co, ro;
    batch_offsets(p, bz, ao, bo, co, ro);
    const float *abase = p.a.p + ao;
    const float *bbase = p.b.p + bo;
    const int kbeg = ks * p.kchunk;
    const int kend = min(p.K, kbeg + p.kchunk);
    const int nk = kend > kbeg ? (kend - kbeg + KSTEP - 1) / KSTEP : 0;

    // ---- DMA source state: row (i * 4 + wave) * 8 + (lane >> 3) of each block --------------
    // Row r keeps k-chunk q at position q ^ f(r) with f(r) = (r & 7) ^ ((r >> 3) & 1): distinct
    // over any 8 consecutive rows and over the 8 even (or odd) rows of any aligned 16, so
    // 16-byte reads of one chunk from 8 or 16 consecutive rows spread over all banks.
    const int q4 = ((lane & 7) ^ (lane >> 3) ^ (wave & 1)) * 4;  // this lane's k offset
    const int rsub = lane >> 3;
    // Operands are read through buffer resources: a masked lane gets an offset past the end of
    // the resource and the hardware returns zeros for it, so no zero page, no select after
    // the load and 32-bit offsets instead of 64-bit addresses.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)abase, (short)0, (int)(p.a_bytes - ao * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)bbase, (short)0, (int)(p.b_bytes - bo * 4), 0x00020000);
    constexpr unsigned OOB = 0x80000000u;  // past every resource's end (extents are < 2^31 bytes)
    // AM_CAT: the second source (batch_rank 0, so no batch offset)
    const __amdgpu_buffer_rsrc_t ra2 = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(AMODE == AM_CAT ? p.a2.p : abase), (short)0, (int)(AMODE == AM_CAT ? p.a2_bytes : 0), 0x00020000);
    unsigned aoff[AI];  // byte offset of the row (AM_VEC) or of its window origin (AM_CONV_VEC)
    unsigned aoff2[AI];  // AM_CAT: byte offset of the row's pixel in the second source
    int aih[AI], aiw[AI];
    const int ohw = AMODE == AM_CAT ? p.a2.OH * p.a2.OW : p.a.OH * p.a.OW;
#pragma unroll
    for (int i = 0; i < AI; ++i) {
        // a quarter's DMA instruction i fetches k block i of the wave's eight rows
        const int m = m0 + (QUARTER ? wave : i * 4 + wave) * 8 + rsub;
        const unsigned kshift = QUARTER ? (unsigned)i * BK * 4u : 0u;
        aoff[i] = aoff2[i] = OOB;
        aih[i] = aiw[i] = -0x40000000;  // fails the window bounds test
        if (m < p.M) {
            if (AMODE == AM_CAT) {
                const int n = fdiv(m, p.div_ohw), rr = m - n * ohw;
                const int oh = fdiv(rr, p.div_ow), ow = rr - oh * p.a2.OW;
                aoff2[i] = (unsigned)(((n * p.a2.H + oh * p.a2.SH) * p.a2.W + ow * p.a2.SW) * p.a2.C) * 4u + kshift;
            }
            if (AMODE == AM_CONV_VEC) {
                const int n = fdiv(m, p.div_ohw), rr = m - n * ohw;
                const int oh = fdiv(rr, p.div_ow), ow = rr - oh * p.a.OW;
                aih[i] = oh * p.a.SH - p.a.PT;
                aiw[i] = ow * p.a.SW - p.a.PL;
                aoff[i] = (unsigned)(((n * p.a.H + aih[i]) * p.a.W + aiw[i]) * p.a.C) * 4u + kshift;
            } else {
                aoff[i] = (unsigned)m * (unsigned)p.a.rs * 4u + kshift;
            }
        }
    }
    unsigned boff[BI];
#pragma unroll
    for (int i = 0; i < BI; ++i) {
        const int n = n0 + (QUARTER ? wave : i * 4 + wave) * 8 + rsub;
        boff[i] = n < p.N ? (unsigned)n * (unsigned)p.b.cs * 4u + (QUARTER ? (unsigned)i * BK * 4u : 0u) : OOB;
    }
    // The lane's next k and, for an image, its (kh, kw, c) split, advanced one stage per issue.
    int knext = kbeg + q4;
    int cc = 0, ckw = 0, ckh = 0;
    if (AMODE == AM_CONV_VEC) {
        const int t = fdiv(knext, p.div_cg);
        cc = knext - t * p.a.cg;
        ckh = fdiv(t, p.div_kw);
        ckw = t - ckh * p.a.KW;
    }

    auto issue = [&](int buf) __attribute__((always_inline)) {
        const int k = knext;
        // k block 1 of a quarter stage starts 32 k later (its offsets carry the shift); a whole
        // tile's stage has one k range (written so that it compiles to the plain form)
        const bool kok0 = k < kend;
        const bool kok1 = QUARTER ? k + BK < kend : kok0;
#define KOK(i) ((QUARTER && (i) == 1) ? kok1 : kok0)
        float *sa = smem + buf * STAGE;
        float *sb = sa + BM * BK;
        if constexpr (AMODE == AM_VEC) {
#pragma unroll
            for (int i = 0; i < AI; ++i)
                dma16_buf(ra, KOK(i) ? aoff[i] + (unsigned)k * 4u : OOB, sa + (i * 4 + wave) * 8 * BK);
        } else if constexpr (AMODE == AM_CAT) {
            // k1 is a multiple of the stage's k (32, or 64 for a quarter tile), so a whole stage
            // reads one source
            if (k < p.k1) {
#pragma unroll
                for (int i = 0; i < AI; ++i)
                    dma16_buf(ra, KOK(i) ? aoff[i] + (unsigned)k * 4u : OOB, sa + (i * 4 + wave) * 8 * BK);
            } else {
                const unsigned k2 = (unsigned)(k - p.k1) * 4u;
#pragma unroll
                for (int i = 0; i < AI; ++i)
                    dma16_buf(ra2, KOK(i) ? aoff2[i] + k2 : OOB, sa + (i * 4 + wave) * 8 * BK);
            }
        } else {
            // a quarter stage's second k block is the same window tap 32 channels on (the
            // channel group is a multiple of 64)
            const int dh = ckh * p.a.DH, dw = ckw * p.a.DW;
            const unsigned koff = (unsigned)((dh * p.a.W + dw) * p.a.C + cc) * 4u;
#pragma unroll
            for (int i = 0; i < AI; ++i) {
                const bool ok = KOK(i) && (unsigned)(aih[i] + dh) < (unsigned)p.a.H &&
                                (unsigned)(aiw[i] + dw) < (unsigned)p.a.W;
                dma16_buf(ra, ok ? aoff[i] + koff : OOB, sa + (i * 4 + wave) * 8 * BK);
            }
            cc += KSTEP;
            while (cc >= p.a.cg) {
                cc -= p.a.cg;
                if (++ckw == p.a.KW) {
                    ckw = 0;
                    ++ckh;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < BI; ++i)
            dma16_buf(rb, KOK(i) ? boff[i] + (unsigned)k * 4u : OOB, sb + (i * 4 + wave) * 8 * BK);
        knext = k + KSTEP;
#undef KOK
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
    const int sw = (li & 7) ^ ((li >> 3) & 1);  // f(row): fragment rows start at multiples of 32

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nk) issue(s);

    constexpr int PER_STAGE = AI + BI;
    for (int kt = 0; kt < nk; ++kt) {
        // Stage kt has landed once at most the later stages' loads are outstanding.
        const int ahead = min(nk - 1 - kt, STAGES - 2);
        if (STAGES >= 4 && ahead >= 2) {
            wait_vmcnt<(STAGES >= 4 ? 2 : 0) * PER_STAGE>();
        } else if (STAGES >= 3 && ahead >= 1) {
            wait_vmcnt<PER_STAGE>();
        } else {
            wait_vmcnt<0>();
        }
        barrier_lds();
        if (kt + STAGES - 1 < nk) issue((kt + STAGES - 1) % STAGES);
        const float *as = smem + (kt % STAGES) * STAGE;
        const float *bs = as + BM * BK;
        if constexpr (QUARTER) {
            // 16 k of k block wave >> 1: chunks (wave & 1) * 4 + lh * 2 + s of rows 32 * kb + li
            const int rq = ((wave >> 1) * 32 + li) * BK;
            const int c0 = (wave & 1) * 4 + lh * 2;
            f4 af[2], bf[2];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                af[s] = *reinterpret_cast<const f4 *>(&as[rq + (((c0 + s) ^ sw) << 2)]);
                bf[s] = *reinterpret_cast<const f4 *>(&bs[rq + (((c0 + s) ^ sw) << 2)]);
            }
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s][e], bf[s][e], acc[0][0], 0, 0, 0);
        } else {
            f4 af[RM][4], bf[RN][4];
#pragma unroll
            for (int i = 0; i < RM; ++i)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    af[i][s] = *reinterpret_cast<const f4 *>(
                        &as[(wm * WM + i * 32 + li) * BK + (((lh * 4 + s) ^ sw) << 2)]);
#pragma unroll
            for (int j = 0; j < RN; ++j)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    bf[j][s] = *reinterpret_cast<const f4 *>(
                        &bs[(wn * WN + j * 32 + li) * BK + (((lh * 4 + s) ^ sw) << 2)]);
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
        }
    }
    __syncthreads();
    if constexpr (QUARTER) {
        // the four waves' partial quarters (pitch 40 floats, 5 KB apart), summed in wave order
        // into the first; register r holds row 8 * (r / 4) + 4 * lh + r % 4, column li
        constexpr int LDQ = 40, PART = 32 * LDQ;
        float *const cw = smem + wave * PART;
#pragma unroll
        for (int r = 0; r < 16; ++r) cw[((r >> 2) * 8 + lh * 4 + (r & 3)) * LDQ + li] = acc[0][0][r];
        __syncthreads();
        const int o = (tid >> 3) * LDQ + (tid & 7) * 4;
        f4 v = *reinterpret_cast<const f4 *>(&smem[o]);
        v += *reinterpret_cast<const f4 *>(&smem[PART + o]);
        v += *reinterpret_cast<const f4 *>(&smem[2 * PART + o]);
        v += *reinterpret_cast<const f4 *>(&smem[3 * PART + o]);
        *reinterpret_cast<f4 *>(&smem[o]) = v;
        __syncthreads();
        gemm_lds_to_global<32, 32>(p, smem, m0, n0, ks, co, ro);
    } else {
        gemm_store_tile<BM, BN, WGM>(p, smem, acc, m0, n0, ks, co, ro);
    }
}

// The 64 x 64 launch with a quarter-tile tail: workgroups below p.nfull take whole tiles, the
// rest take quarters of the tiles after them (four workgroups per tile), so a tile count just
// past a multiple of the CU count does not leave a few CUs running one more whole tile than the
// others. Within each range consecutive tiles go to one XCD (the hardware deals workgroup ids
// round-robin to the eight XCDs), which keeps a tile row's A block in one L2. Launches without
// such a tail run gemm_dma_kernel: its whole tiles compile to a tighter K loop than this
// kernel's shared body (measured 2-4% faster per launch).
template <int AMODE>
__global__ void __launch_bounds__(256) gemm_dma_tail_kernel(const GemmDev p) {
    constexpr int BM = 64, BN = 64, WGM = 2, STAGES = 2;
    __shared__ __attribute__((aligned(16))) float smem[dma_smem_floats<BM, BN, STAGES>()];
    const int nb = gridDim.x;
    const int nfull = p.nfull < nb ? p.nfull : nb;
    int lin = blockIdx.x;
    const bool quarter = lin >= nfull;
    const int first = quarter ? nfull : 0;
    const int span = (quarter ? nb - nfull : nfull) & ~7;
    lin -= first;
    if (lin < span) {
        const int per = span >> 3;
        lin = (lin & 7) * per + (lin >> 3);
    }
    if (quarter) {
        const int t = nfull + (lin >> 2);
        const int tm = t / p.tiles_n;
        const int tn = t - tm * p.tiles_n;
        gemm_dma_tile<BM, BN, WGM, STAGES, AMODE, true>(p, smem, tm * BM + (lin & 1) * 32,
                                                       tn * BN + ((lin >> 1) & 1) * 32);
        return;
    }
    const int tm = lin / p.tiles_n;
    const int tn = lin - tm * p.tiles_n;
    gemm_dma_tile<BM, BN, WGM, STAGES, AMODE, false>(p, smem, tm * BM, tn * BN);
}

// GEMM / implicit-GEMM convolution on 32 x 32 output tiles whose K range is dealt out to the
// workgroup's four waves (wave w takes the 32-wide K stages w, w + 4, ...), each with its own
// two-stage DMA ring in LDS; the four partial tiles are summed through LDS in wave order, each
// thread adding the 16-byte chunk whose bias and residual it requested when the kernel started
// (their latency overlaps the K loop). For GEMMs whose 64 x 64 tiles are too few to occupy the CUs (small M at
// batch 1), where the alternative is a K split over workgroups and a second kernel that adds
// the partials: this kernel spreads the same work over four times as many tiles and finishes
// in one launch. The waves synchronise only around the epilogue; in the main loop each wave
// waits for its own loads (s_waitcnt), since it alone reads what it loaded. Operand forms as
// gemm_dma_kernel (k-contiguous A or an NHWC image, packed [N][K] B). Row r of a wave's
// 32-row block keeps k-chunk q at position q ^ (r & 7), so the eight lanes that read one chunk
// of eight consecutive rows hit eight different positions.
template <int AMODE>
__global__ void __launch_bounds__(256) gemm_dma_wsplit_kernel(const GemmDev p) {
    constexpr int BK = 32, T = 32;
    constexpr int STAGE = 2 * T * BK;  // one wave's A and B blocks of one stage (floats)
    constexpr int RING = 2 * STAGE;    // two stages per wave
    constexpr int LDC = T + 8;
    constexpr int SMEM = 4 * RING;     // 64 KB; the epilogue uses 4 * T * LDC floats of it
    static_assert(4 * T * LDC <= SMEM, "epilogue staging");
    static_assert(AMODE == AM_VEC || AMODE == AM_CONV_VEC || AMODE == AM_CAT, "vector A only");

    __shared__ __attribute__((aligned(16))) float smem[SMEM];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const int nb = gridDim.x;
    const int full = nb & ~7;
    int lin = blockIdx.x;
    if (lin < full) {
        const int per = full >> 3;
        lin = (lin & 7) * per + (lin >> 3);
    }
    const int tm = lin / p.tiles_n;
    const int tn = lin - tm * p.tiles_n;
    const int m0 = tm * T, n0 = tn * T;

    const int bz = blockIdx.z / p.split;
    const int ks = blockIdx.z - bz * p.split;
    long ao, bo, co, ro;
    batch_offsets(p, bz, ao, bo, co, ro);

    // epilogue operands first: thread t owns row t / 8, columns 4 (t % 8) .. + 3
    const bool split_out = p.split > 1;
    const int er = tid >> 3, ec = (tid & 7) * 4;
    const int erow = m0 + er, ecol = n0 + ec;
    const bool eok = erow < p.M && ecol < p.N;
    const bool efull = eok && ecol + 4 <= p.N && (split_out ? (p.N % 4 == 0) : p.vec_out != 0);
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
    f4 ebias = zero4, eres = zero4;
    if (efull && !split_out) {
        if (p.bias && p.bias_mode == 1) ebias = ldg4(p.bias + ecol);
        if (p.res) eres = ldg4(p.res + ro + (long)erow * p.ldr + ecol);
    }

    const float *abase = p.a.p + ao;
    const float *bbase = p.b.p + bo;
    const int kbeg = ks * p.kchunk;
    const int kend = min(p.K, kbeg + p.kchunk);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int nkw = nk > wave ? (nk - 1 - wave) / 4 + 1 : 0;  // this wave's stages

    const int rsub = lane >> 3;
    const int q4 = ((lane & 7) ^ rsub) * 4;  // this lane's k offset within a stage
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)abase, (short)0, (int)(p.a_bytes - ao * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)bbase, (short)0, (int)(p.b_bytes - bo * 4), 0x00020000);
    constexpr unsigned OOB = 0x80000000u;
    const __amdgpu_buffer_rsrc_t ra2 = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(AMODE == AM_CAT ? p.a2.p : abase), (short)0, (int)(AMODE == AM_CAT ? p.a2_bytes : 0), 0x00020000);
    unsigned aoff[4], aoff2[4];
    int aih[4], aiw[4];
    const int ohw = AMODE == AM_CAT ? p.a2.OH * p.a2.OW : p.a.OH * p.a.OW;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + i * 8 + rsub;
        aoff[i] = aoff2[i] = OOB;
        aih[i] = aiw[i] = -0x40000000;
        if (m < p.M) {
            if (AMODE == AM_CAT) {
                const int n = fdiv(m, p.div_ohw), rr = m - n * ohw;
                const int oh = fdiv(rr, p.div_ow), ow = rr - oh * p.a2.OW;
                aoff2[i] = (unsigned)(((n * p.a2.H + oh * p.a2.SH) * p.a2.W + ow * p.a2.SW) * p.a2.C) * 4u;
            }
            if (AMODE == AM_CONV_VEC) {
                const int n = fdiv(m, p.div_ohw), rr = m - n * ohw;
                const int oh = fdiv(rr, p.div_ow), ow = rr - oh * p.a.OW;
                aih[i] = oh * p.a.SH - p.a.PT;
                aiw[i] = ow * p.a.SW - p.a.PL;
                aoff[i] = (unsigned)(((n * p.a.H + aih[i]) * p.a.W + aiw[i]) * p.a.C) * 4u;
            } else {
                aoff[i] = (unsigned)m * (unsigned)p.a.rs * 4u;
            }
        }
    }
    unsigned boff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = n0 + i * 8 + rsub;
        boff[i] = n < p.N ? (unsigned)n * (unsigned)p.b.cs * 4u : OOB;
    }
    int knext = kbeg + wave * BK + q4;
    int cc = 0, ckw = 0, ckh = 0;
    if (AMODE == AM_CONV_VEC) {
        const int t = fdiv(knext, p.div_cg);
        cc = knext - t * p.a.cg;
        ckh = fdiv(t, p.div_kw);
        ckw = t - ckh * p.a.KW;
    }
    float *const ring = smem + wave * RING;

    auto issue = [&](int buf) __attribute__((always_inline)) {
        const int k = knext;
        const bool kok = k < kend;
        float *sa = ring + buf * STAGE;
        float *sb = sa + T * BK;
        if constexpr (AMODE == AM_VEC) {
#pragma unroll
            for (int i = 0; i < 4; ++i) dma16_buf(ra, kok ? aoff[i] + (unsigned)k * 4u : OOB, sa + i * 8 * BK);
        } else if constexpr (AMODE == AM_CAT) {
            if (k < p.k1) {
#pragma unroll
                for (int i = 0; i < 4; ++i) dma16_buf(ra, kok ? aoff[i] + (unsigned)k * 4u : OOB, sa + i * 8 * BK);
            } else {
                const unsigned k2 = (unsigned)(k - p.k1) * 4u;
#pragma unroll
                for (int i = 0; i < 4; ++i) dma16_buf(ra2, kok ? aoff2[i] + k2 : OOB, sa + i * 8 * BK);
            }
        } else {
            const int dh = ckh * p.a.DH, dw = ckw * p.a.DW;
            const unsigned koff = (unsigned)((dh * p.a.W + dw) * p.a.C + cc) * 4u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool ok = kok && (unsigned)(aih[i] + dh) < (unsigned)p.a.H &&
                                (unsigned)(aiw[i] + dw) < (unsigned)p.a.W;
                dma16_buf(ra, ok ? aoff[i] + koff : OOB, sa + i * 8 * BK);
            }
            cc += 4 * BK;
            while (cc >= p.a.cg) {
                cc -= p.a.cg;
                if (++ckw == p.a.KW) {
                    ckw = 0;
                    ++ckh;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16_buf(rb, kok ? boff[i] + (unsigned)k * 4u : OOB, sb + i * 8 * BK);
        knext = k + 4 * BK;
    };

    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    const int li = lane & 31;
    const int lh = lane >> 5;
    const int sw = li & 7;

    if (nkw > 0) issue(0);
    for (int kt = 0; kt < nkw; ++kt) {
        // this wave's stage kt has landed in LDS; its reads of the other buffer (stage kt - 1)
        // are complete before the next stage's DMA overwrites it
        wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (kt + 1 < nkw) issue((kt + 1) & 1);
        const float *as = ring + (kt & 1) * STAGE;
        const float *bs = as + T * BK;
        f4 af[4], bf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            af[s] = *reinterpret_cast<const f4 *>(&as[li * BK + (((lh * 4 + s) ^ sw) << 2)]);
            bf[s] = *reinterpret_cast<const f4 *>(&bs[li * BK + (((lh * 4 + s) ^ sw) << 2)]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s][e], bf[s][e], acc, 0, 0, 0);
    }
    __syncthreads();
    // partial tiles -> LDS slots (register r of a 32 x 32 block holds row 8 (r / 4) + 4 lh + r % 4,
    // column li), then each thread adds one 16-byte chunk of the four slots in wave order
    float *const slot = smem + wave * (T * LDC);
#pragma unroll
    for (int r = 0; r < 16; ++r) slot[((r >> 2) * 8 + lh * 4 + (r & 3)) * LDC + li] = acc[r];
    __syncthreads();
    if (!eok) return;
    const int o = er * LDC + ec;
    f4 v = *reinterpret_cast<const f4 *>(&smem[o]);
    v += *reinterpret_cast<const f4 *>(&smem[T * LDC + o]);
    v += *reinterpret_cast<const f4 *>(&smem[2 * T * LDC + o]);
    v += *reinterpret_cast<const f4 *>(&smem[3 * T * LDC + o]);
    const int ncol = min(4, p.N - ecol);
    if (split_out) {
        float *dst = p.ws + (long)ks * p.M * p.N + (long)erow * p.N + ecol;
        if (efull) {
            *reinterpret_cast<f4 *>(dst) = v;
        } else {
            for (int e = 0; e < ncol; ++e) dst[e] = v[e];
        }
        return;
    }
    if (!efull) {  // scalar bias and residual reads
        for (int e = 0; e < ncol; ++e) {
            if (p.bias && p.bias_mode == 1) ebias[e] = ldg(p.bias + ecol + e);
            if (p.res) eres[e] = ldg(p.res + ro + (long)erow * p.ldr + ecol + e);
        }
    }
    v = v * p.alpha + ebias;
    if (p.bias && p.bias_mode == 2) v += ldg(p.bias + erow);
    if (p.res) v += p.beta * eres;
    v = act4(v, p.act, p.lo, p.hi);
    float *dst = p.c + co + (long)erow * p.ldc + ecol;
    if (efull) {
        *reinterpret_cast<f4 *>(dst) = v;
    } else {
        for (int e = 0; e < ncol; ++e) dst[e] = v[e];
    }
}

// vmcnt wait for a count known only at run time (0 <= n < 8 stages of PER loads each).
template <int PER>
__device__ __forceinline__ void wait_stages(int n) {
    switch (n) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<PER>(); break;
    case 2: wait_vmcnt<2 * PER>(); break;
    case 3: wait_vmcnt<3 * PER>(); break;
    case 4: wait_vmcnt<4 * PER>(); break;
    case 5: wait_vmcnt<5 * PER>(); break;
    case 6: wait_vmcnt<6 * PER>(); break;
    default: wait_vmcnt<7 * PER>(); break;
    }
}

// Epilogue of the 16 x 16 wave-split kernels: each wave's partial tile (register r of acc holds
// row 4 (lane / 16) + r, column lane % 16) goes to its LDS slot (smem holds at least
// WAVES * 16 * 20 floats, free when this is called), and thread t < 64 sums the slots' chunk
// (row t / 4, columns 4 (t % 4) .. + 3) in wave order, applies alpha, bias, residual and
// activation (its bias and residual chunks requested by the caller before the K loop) and stores
// it, or writes the raw sum to the K-split workspace.
template <int WAVES>
__device__ __forceinline__ void wsplit16_finish(const GemmDev &p, float *smem, const f4 acc, int tid, int ks,
                                                long co, long ro, bool split_out, int er, int ec, int erow,
                                                int ecol, bool eok, bool efull, const f4 &ebias, const f4 &eres) {
    constexpr int T = 16, LDC = T + 4;
    // the argument block's fields read once into registers (a reference into the kernel's
    // argument block kept live across the epilogue makes the compiler copy it to scratch)
    const int M = p.M, N = p.N, act = p.act, bias_mode = p.bias ? p.bias_mode : 0;
    const float alpha = p.alpha, beta = p.beta, lo = p.lo, hi = p.hi;
    const float *const bias = p.bias;
    const float *const res = p.res;
    float *const ws = p.ws;
    float *const c = p.c;
    const long ldr = p.ldr, ldc = p.ldc;
    const int lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    float *const slot = smem + wave * (T * LDC);
#pragma unroll
    for (int r = 0; r < 4; ++r) slot[(4 * lg + r) * LDC + li] = acc[r];
    __syncthreads();
    if (!eok) return;
    const int o = er * LDC + ec;
    f4 v = *reinterpret_cast<const f4 *>(&smem[o]);
#pragma unroll
    for (int w = 1; w < WAVES; ++w) v += *reinterpret_cast<const f4 *>(&smem[w * T * LDC + o]);
    const int ncol = min(4, N - ecol);
    // a partial chunk (the last columns of an N that is not a multiple of 4, or unaligned
    // rows) goes element by element
    auto store = [&](float *dst) __attribute__((always_inline)) {
        if (efull) {
            *reinterpret_cast<f4 *>(dst) = v;
        } else {
            dst[0] = v[0];
            if (ncol > 1) dst[1] = v[1];
            if (ncol > 2) dst[2] = v[2];
            if (ncol > 3) dst[3] = v[3];
        }
    };
    if (split_out) {
        store(ws + (long)ks * M * N + (long)erow * N + ecol);
        return;
    }
    f4 b = ebias, r = eres;
    if (!efull) {  // scalar bias and residual reads
        const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
        b = zero4;
        r = zero4;
        if (bias_mode == 1) {
            const float *bp = bias + ecol;
            b[0] = ldg(bp);
            if (ncol > 1) b[1] = ldg(bp + 1);
            if (ncol > 2) b[2] = ldg(bp + 2);
            if (ncol > 3) b[3] = ldg(bp + 3);
        }
        if (res) {
            const float *rp = res + ro + (long)erow * ldr + ecol;
            r[0] = ldg(rp);
            if (ncol > 1) r[1] = ldg(rp + 1);
            if (ncol > 2) r[2] = ldg(rp + 2);
            if (ncol > 3) r[3] = ldg(rp + 3);
        }
    }
    v = v * alpha + b;
    if (bias_mode == 2) v += ldg(bias + erow);
    if (res) v += beta * r;
    v = act4(v, act, lo, hi);
    store(c + co + (long)erow * ldc + ecol);
}

// GEMM / implicit-GEMM convolution on 16 x 16 output tiles whose K range is dealt out to the
// workgroup's WAVES waves (wave w takes the 32-wide K stages w, w + WAVES, ...), each with a
// STAGES-deep DMA ring of its own, on v_mfma_f32_16x16x4f32 (the 32 x 32 x 2 form's rate per
// SIMD). For batch-1 layers whose 32 x 32 tiles are too few for the CUs even with their K dealt
// to four waves: a 14 x 14 image with 256 output channels has 56 tiles of 32 x 32 and 208 of
// 16 x 16, so the latter needs no K split over workgroups and no reduction launch. A stage is
// a quarter of a 32 x 32 stage's MFMA work; with eight waves two share each SIMD, so one
// multiplies while the other waits for its loads.
// Operand forms as gemm_dma_wsplit_kernel; row r of a 16-row block keeps k-chunk q at LDS
// position q ^ (r & 7).
//
// The k order inside a stage is permuted: lane group g = lane / 16 reads chunks 2g and 2g + 1
// (k = 8g .. 8g + 7) of its row and MFMA j takes element j of those eight, so instruction j
// multiplies A[:, 8g + j] by B[8g + j, :] over the four groups; A and B use the same
// permutation, and the eight instructions cover the stage's 32 k once. Register r of the
// 16 x 16 accumulator holds row 4 (lane / 16) + r, column lane % 16.
//
// The epilogue's bias and residual chunks are requested before the main loop, so their latency
// overlaps the K loop instead of following it.
template <int AMODE, int STAGES, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) gemm_dma_wsplit16_kernel(const GemmDev p) {
    constexpr int BK = 32, T = 16;
    constexpr int STAGE = 2 * T * BK;  // one wave's A and B blocks of one stage (floats)
    constexpr int RING = STAGES * STAGE;
    constexpr int LDC = T + 4;
    constexpr int SMEM = WAVES * RING;
    constexpr int PER = 4;  // DMA loads per lane per stage (two A, two B)
    static_assert(WAVES * T * LDC <= SMEM, "epilogue staging");
    static_assert(STAGES >= 2 && STAGES <= 8, "stages");
    static_assert(AMODE == AM_VEC || AMODE == AM_CONV_VEC || AMODE == AM_CAT, "vector A only");

    __shared__ __attribute__((aligned(16))) float smem[SMEM];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const int nb = gridDim.x;
    const int full = nb & ~7;
    int lin = blockIdx.x;
    if (lin < full) {  // consecutive tiles (which share A rows) on one XCD
        const int per = full >> 3;
        lin = (lin & 7) * per + (lin >> 3);
    }
    const int tm = lin / p.tiles_n;
    const int tn = lin - tm * p.tiles_n;
    const int m0 = tm * T, n0 = tn * T;

    const int bz = blockIdx.z / p.split;
    const int ks = blockIdx.z - bz * p.split;
    long ao, bo, co, ro;
    batch_offsets(p, bz, ao, bo, co, ro);

    // ---- epilogue operands first (thread t < 64: row t / 4, columns 4 (t % 4) .. + 3) ------
    const bool split_out = p.split > 1;
    const int er = tid >> 2, ec = (tid & 3) * 4;
    const int erow = m0 + er, ecol = n0 + ec;
    const bool eok = tid < 64 && erow < p.M && ecol < p.N;
    const bool efull = eok && ecol + 4 <= p.N && (split_out ? (p.N % 4 == 0) : p.vec_out != 0);
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
    f4 ebias = zero4, eres = zero4;
    if (efull && !split_out) {
        if (p.bias && p.bias_mode == 1) ebias = ldg4(p.bias + ecol);
        if (p.res) eres = ldg4(p.res + ro + (long)erow * p.ldr + ecol);
    }

    const float *abase = p.a.p + ao;
    const float *bbase = p.b.p + bo;
    const int kbeg = ks * p.kchunk;
    const int kend = min(p.K, kbeg + p.kchunk);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int nkw = nk > wave ? (nk - 1 - wave) / WAVES + 1 : 0;  // this wave's stages

    const int rsub = lane >> 3;
    const int q4 = ((lane & 7) ^ rsub) * 4;  // this lane's k offset within a stage
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)abase, (short)0, (int)(p.a_bytes - ao * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)bbase, (short)0, (int)(p.b_bytes - bo * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t ra2 = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(AMODE == AM_CAT ? p.a2.p : abase), (short)0, (int)(AMODE == AM_CAT ? p.a2_bytes : 0), 0x00020000);
    constexpr unsigned OOB = 0x80000000u;
    unsigned aoff[2], aoff2[2], boff[2];
    int aih[2], aiw[2];
    const int ohw = AMODE == AM_CAT ? p.a2.OH * p.a2.OW : p.a.OH * p.a.OW;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = m0 + i * 8 + rsub;
        aoff[i] = aoff2[i] = OOB;
        aih[i] = aiw[i] = -0x40000000;
        if (m < p.M) {
            if (AMODE == AM_CAT) {
                const int n = fdiv(m, p.div_ohw), rr = m - n * ohw;
                const int oh = fdiv(rr, p.div_ow), ow = rr - oh * p.a2.OW;
                aoff2[i] = (unsigned)(((n * p.a2.H + oh * p.a2.SH) * p.a2.W + ow * p.a2.SW) * p.a2.C) * 4u;
            }
            if (AMODE == AM_CONV_VEC) {
                const int n = fdiv(m, p.div_ohw), rr = m - n * ohw;
                const int oh = fdiv(rr, p.div_ow), ow = rr - oh * p.a.OW;
                aih[i] = oh * p.a.SH - p.a.PT;
                aiw[i] = ow * p.a.SW - p.a.PL;
                aoff[i] = (unsigned)(((n * p.a.H + aih[i]) * p.a.W + aiw[i]) * p.a.C) * 4u;
            } else {
                aoff[i] = (unsigned)m * (unsigned)p.a.rs * 4u;
            }
        }
        const int n = n0 + i * 8 + rsub;
        boff[i] = n < p.N ? (unsigned)n * (unsigned)p.b.cs * 4u : OOB;
    }
    int knext = kbeg + wave * BK + q4;
    int cc = 0, ckw = 0, ckh = 0;
    if (AMODE == AM_CONV_VEC) {
        const int t = fdiv(knext, p.div_cg);
        cc = knext - t * p.a.cg;
        ckh = fdiv(t, p.div_kw);
        ckw = t - ckh * p.a.KW;
    }
    float *const ring = smem + wave * RING;

    auto issue = [&](int buf) __attribute__((always_inline)) {
        const int k = knext;
        const bool kok = k < kend;
        float *sa = ring + buf * STAGE;
        float *sb = sa + T * BK;
        if constexpr (AMODE == AM_VEC) {
#pragma unroll
            for (int i = 0; i < 2; ++i) dma16_buf(ra, kok ? aoff[i] + (unsigned)k * 4u : OOB, sa + i * 8 * BK);
        } else if constexpr (AMODE == AM_CAT) {
            // k1 is a multiple of 32, so a whole stage reads one source
            if (k < p.k1) {
#pragma unroll
                for (int i = 0; i < 2; ++i) dma16_buf(ra, kok ? aoff[i] + (unsigned)k * 4u : OOB, sa + i * 8 * BK);
            } else {
                const unsigned k2 = (unsigned)(k - p.k1) * 4u;
#pragma unroll
                for (int i = 0; i < 2; ++i) dma16_buf(ra2, kok ? aoff2[i] + k2 : OOB, sa + i * 8 * BK);
            }
        } else {
            const int dh = ckh * p.a.DH, dw = ckw * p.a.DW;
            const unsigned koff = (unsigned)((dh * p.a.W + dw) * p.a.C + cc) * 4u;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const bool ok = kok && (unsigned)(aih[i] + dh) < (unsigned)p.a.H &&
                                (unsigned)(aiw[i] + dw) < (unsigned)p.a.W;
                dma16_buf(ra, ok ? aoff[i] + koff : OOB, sa + i * 8 * BK);
            }
            cc += WAVES * BK;
            while (cc >= p.a.cg) {
                cc -= p.a.cg;
                if (++ckw == p.a.KW) {
                    ckw = 0;
                    ++ckh;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16_buf(rb, kok ? boff[i] + (unsigned)k * 4u : OOB, sb + i * 8 * BK);
        knext = k + WAVES * BK;
    };

    f4 acc = zero4;
    const int li = lane & 15;
    const int lg = lane >> 4;
    const int sw = li & 7;
    const int pa = li * BK + (((2 * lg) ^ sw) << 2);      // chunk 2g of row li
    const int pb = li * BK + (((2 * lg + 1) ^ sw) << 2);  // chunk 2g + 1

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nkw) issue(s);
    for (int kt = 0; kt < nkw; ++kt) {
        // stage kt has landed once at most the later stages' loads are outstanding; this wave's
        // reads of the buffer the next issue overwrites (stage kt - 1) are complete
        wait_stages<PER>(min(nkw - 1 - kt, STAGES - 2));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (kt + STAGES - 1 < nkw) issue((kt + STAGES - 1) % STAGES);
        const float *as = ring + (kt % STAGES) * STAGE;
        const float *bs = as + T * BK;
        const f4 a0 = *reinterpret_cast<const f4 *>(&as[pa]);
        const f4 a1 = *reinterpret_cast<const f4 *>(&as[pb]);
        const f4 b0 = *reinterpret_cast<const f4 *>(&bs[pa]);
        const f4 b1 = *reinterpret_cast<const f4 *>(&bs[pb]);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[e], b0[e], acc, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[e], b1[e], acc, 0, 0, 0);
    }
    __syncthreads();  // every wave is done with its ring (the slots below overlap the rings)
    wsplit16_finish<WAVES>(p, smem, acc, tid, ks, co, ro, split_out, er, ec, erow, ecol, eok, efull, ebias, eres);
}

// GEMMs with short K (K <= 2 * KH, KH 8 or 16, K % 4 == 0) over many rows: the expand and
// project 1 x 1 convolutions of MobileNet-style blocks at large batch, which move tens of MB
// per launch for a few FLOP per byte and so are HBM-bound. The tiled kernels spend most of such
// a launch on per-workgroup latency (load, multiply, stage through LDS, store, one tile per
// workgroup). Here each wave streams 32-row tiles on its own: A goes straight from memory into
// registers (a tile's rows are contiguous, 32 x K floats), the next tile's A is requested before
// this tile's MFMAs (two register sets used in turn), the wave's column group of B (NB blocks of
// 32 columns) stays in registers for all its tiles, and the epilogue writes from the
// accumulators (no LDS, no barriers). Lane (li, h) = (lane % 32, lane / 32) holds k = KH h ..
// KH h + KH - 1 of row li (A) and of column li (B), and MFMA j multiplies A[:, KH h + j] by
// B[KH h + j, :] over both halves, so the KH instructions cover the 2 KH k once; register r of a
// 32 x 32 accumulator holds row 8 (r / 4) + 4 h + r % 4, column li. Every operand goes through
// a buffer resource: columns of B past N, k past K and rows of A past M load as zeros (so the
// padding multiplies 0 by 0), and C and residual accesses past M or N are dropped, which keeps
// the epilogue free of branches. Activation relu or clip as one clamp to [lo, hi] (lo = 0,
// hi = +inf for relu: fmaxf maps NaN to 0 as relu's v > 0 ? v : 0 does); none stores v unchanged
// (clamp = 0, a uniform test), so NaN passes through as in every other epilogue. Waves are dealt
// to column groups, wave w of a group taking M-tiles w, w + waves_per_group, ...
// CONV: A is an NHWC image read through its implicit im2col (one channel group, C % 4 == 0, so
// a lane's 16-byte quads never straddle two window taps): a row is an output pixel, and lane
// (li, h) reads its KH k of the window (tap k / C, channel k % C) straight from the image, taps
// outside the image as zeros. MobileNetV2's stem (a 3 x 3 stride-2 convolution over three
// channels, run as a 2 x 2 convolution over its space-to-depth copy: K = 48) streams this way.
template <int KH, int NB, bool CONV>
__global__ void __launch_bounds__(256) gemm_stream_kernel(const GemmDev p, int groups, int waves_per_group,
                                                          int clamp, float lo, float hi, long c_bytes, long r_bytes) {
    const int lane = threadIdx.x & 63, li = lane & 31, h = lane >> 5;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= groups * waves_per_group) return;
    const int grp = gw % groups;
    const int tiles_m = (p.M + 31) / 32;
    const int n0 = grp * NB * 32;
    const int kh0 = KH * h;  // this lane's first k
    constexpr int Q = KH / 4;
    constexpr unsigned OOB = 0x80000000u;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)p.a.p, (short)0, (int)p.a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void *)p.b.p, (short)0, (int)p.b_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc((void *)p.c, (short)0, (int)c_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc((void *)(p.res ? p.res : p.c), (short)0,
                                                                        (int)(p.res ? r_bytes : 0), 0x00020000);
    const bool has_res = p.res != nullptr;
    const float alpha = p.alpha, beta = p.beta;
    bool kok[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) kok[q] = kh0 + 4 * q < p.K;

    f4 b[NB][Q];
    float bias[NB];
    unsigned cofs[NB], rofs[NB];  // byte offsets of this lane's column in C / R (row 0), or OOB
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int n = n0 + nb * 32 + li;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const unsigned off = n < p.N && kok[q] ? ((unsigned)n * (unsigned)p.b.cs + kh0 + 4 * q) * 4u : OOB;
            b[nb][q] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
        }
        bias[nb] = p.bias && n < p.N ? ldg(p.bias + n) : 0.0f;
        cofs[nb] = n < p.N ? (unsigned)n * 4u : OOB;
        rofs[nb] = n < p.N ? (unsigned)n * 4u : OOB;
    }
    const unsigned ldc4 = (unsigned)p.ldc * 4u, ldr4 = (unsigned)p.ldr * 4u;

    // CONV: the window tap (dy, dx) and channel of each of this lane's quads
    int tdy[Q], tdx[Q], tch[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        tdy[q] = tdx[q] = tch[q] = 0;
        if (CONV) {
            const int k = kh0 + 4 * q;
            const int t = k / p.a.C;
            tch[q] = k - t * p.a.C;
            tdy[q] = (t / p.a.KW) * p.a.DH;
            tdx[q] = (t - (t / p.a.KW) * p.a.KW) * p.a.DW;
        }
    }
    auto load_a = [&](f4 (&a)[Q], int tm) __attribute__((always_inline)) {
        const int row = tm * 32 + li;
        if (CONV) {
            const int rr = row < p.M ? row : 0;
            const int n = fdiv(rr, p.div_ohw), rem = rr - n * (p.a.OH * p.a.OW);
            const int oh = fdiv(rem, p.div_ow), ow = rem - oh * p.a.OW;
            const int ih0 = oh * p.a.SH - p.a.PT, iw0 = ow * p.a.SW - p.a.PL;
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const int ih = ih0 + tdy[q], iw = iw0 + tdx[q];
                const bool ok = row < p.M && kok[q] && (unsigned)ih < (unsigned)p.a.H && (unsigned)iw < (unsigned)p.a.W;
                const unsigned off =
                    ok ? ((unsigned)((n * p.a.H + ih) * p.a.W + iw) * (unsigned)p.a.C + (unsigned)tch[q]) * 4u : OOB;
                a[q] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
            }
        } else {
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const unsigned off = row < p.M && kok[q] ? ((unsigned)row * (unsigned)p.a.rs + kh0 + 4 * q) * 4u : OOB;
                a[q] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
            }
        }
    };
    auto tile = [&](const f4 (&a)[Q], int tm) __attribute__((always_inline)) {
        floatx16 acc[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[nb][r] = 0.0f;
#pragma unroll
        for (int j = 0; j < KH; ++j)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                acc[nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j >> 2][j & 3], b[nb][j >> 2][j & 3], acc[nb], 0, 0, 0);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            unsigned rowofs[16];
            float res[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = tm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                rowofs[r] = row < p.M ? (unsigned)row : OOB;
                res[r] = 0.0f;
            }
            if (has_res) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const unsigned off = rowofs[r] == OOB || rofs[nb] == OOB ? OOB : rowofs[r] * ldr4 + rofs[nb];
                    res[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, off, 0, 0));
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float v = acc[nb][r] * alpha + bias[nb] + beta * res[r];
                if (clamp) v = fminf(fmaxf(v, lo), hi);
                const unsigned off = rowofs[r] == OOB || cofs[nb] == OOB ? OOB : rowofs[r] * ldc4 + cofs[nb];
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), rc, off, 0, 0);
            }
        }
    };

    f4 a0[Q], a1[Q];
    int tm = gw / groups;
    if (tm < tiles_m) load_a(a0, tm);
    while (tm < tiles_m) {
        const int t1 = tm + waves_per_group;
        if (t1 < tiles_m) load_a(a1, t1);
        tile(a0, tm);
        if (t1 >= tiles_m) break;
        const int t2 = t1 + waves_per_group;
        if (t2 < tiles_m) load_a(a0, t2);
        tile(a1, t1);
        tm = t2;
    }
}

// A depthwise 3 x 3 convolution computed inside the GEMM of the 1 x 1 convolution that reads it
// (mgc_hip_gemm_dw): A[m][k] = act_d(bd[k] + sum_{i,j} X[n, oh SH - PT + i, ow SW - PL + j, k]
// wd[(3 i + j) C + k]) for output pixel m = (n, oh, ow) and channel k, evaluated while the A tile
// is staged, so the depthwise output never goes to memory. The taps are summed in the order of
// the standalone depthwise kernel (bias first, then row by row), so A holds exactly the values
// that kernel would store.
struct DwDev {
    const float *x, *w, *bias;
    int H, W, C, PT, PL, OH, OW;
    int act;
    float lo, hi;
    int tiles_h, tiles_w;  // 8 x 8 output-pixel tiles per image
    long x_bytes;          // bytes of x reachable from d.x
};

// One workgroup (256 threads) computes an 8 x 8 block of output pixels of one image (64 GEMM
// rows) times BN output channels; K runs over the depthwise channels in stages of 32.
//  * Per stage the input patch the 64 depthwise windows cover ((7 S + 3)^2 pixels x 32 channels)
//    travels to LDS by DMA (buffer_load ... lds, 16 bytes per lane, zeros outside the image and
//    past C), each element once; the depthwise weights, bias and the B quads of the stage come
//    into registers one stage ahead. With PBUF 2 the patch is double-buffered (its DMA for the
//    next stage runs under this stage's depthwise and MFMA work); with PBUF 1 the next patch is
//    requested after the depthwise pass (less LDS, more workgroups per CU).
//  * Thread t computes channel quad t & 7 of tile rows t >> 3 and (t >> 3) + 32 (row r is pixel
//    (r >> 3, r & 7) of the block) from the patch into the A tile. BN 64: 2 x 2 waves of 32 x 32
//    MFMA blocks; BN 32: waves w and w + 2 share the 32 x 32 block of rows 32 w, taking k 0-15
//    and 16-31 of each stage, and sum their halves through LDS at the end.
//  * The A and B tiles keep 32-float rows with the quads XOR-swizzled (no padding): the stride-1
//    form then takes 38 KB of LDS for BN 32, so four workgroups fit a CU (the CU's 160 KB hold
//    four of 40 KB only in the occupancy query, not on the hardware).
//  * The epilogue maps tile rows back to pixels (rows outside the image are not stored).
template <int BN, int S, int PBUF>
__global__ void __launch_bounds__(256) gemm_dw_kernel(const GemmDev p, const DwDev d) {
    constexpr int BM = 64;
    constexpr int BK = 32;
    constexpr int LDK = BK;  // rows unpadded: quad q of row r sits at position q ^ f(r)
    constexpr int PWID = 7 * S + 3;                    // patch rows and columns
    constexpr int PQUADS = PWID * PWID * 8;             // 16-byte quads of one patch
    constexpr int PINS = (PQUADS + 63) / 64;            // DMA instructions per patch
    constexpr int PIW = (PINS + 3) / 4;                 // per wave
    constexpr int PFLOATS = PINS * 64 * 4;              // one patch buffer, whole instructions
    constexpr int BV = BN / 32;
    constexpr int LDC = BN + 8;
    constexpr int SMEM_LOOP = PBUF * PFLOATS + BM * LDK + BN * LDK;
    constexpr int SMEM_EPI = BM * LDC + (BN == 32 ? 2 * 1024 : 0);
    constexpr int SMEM = SMEM_LOOP > SMEM_EPI ? SMEM_LOOP : SMEM_EPI;
    static_assert(BN == 32 || BN == 64, "tile");
    static_assert(S == 1 || S == 2, "stride");
    static_assert(PBUF == 1 || PBUF == 2, "patch buffers");

    __shared__ __attribute__((aligned(16))) float smem[SMEM];
    float *const Ps = smem;                          // [PBUF][PFLOATS] patches [pixel][32]
    float *const As = smem + PBUF * PFLOATS;         // [BM][32], swizzled
    float *const Bs = As + BM * LDK;                 // [BN][32], swizzled
    // f(r) = (r & 7) ^ ((r >> 3) & 1): distinct over any 8 consecutive rows and over the 8 even
    // (or odd) rows of an aligned 16, so 16-byte reads of one quad from 8 or 16 rows spread over
    // the banks (the layout of gemm_dma_kernel's stages)
    auto swz = [](int r) __attribute__((always_inline)) { return (r & 7) ^ ((r >> 3) & 1); };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = BN == 64 ? wave >> 1 : wave & 1;
    const int wn = BN == 64 ? wave & 1 : 0;
    const int khalf = BN == 64 ? 0 : wave >> 1;

    // tile order: XCD-aware, output-channel tiles of one pixel block adjacent (they read the
    // same patches)
    const int nb = gridDim.x;
    const int full = nb & ~7;
    int lin = blockIdx.x;
    if (lin < full) {
        const int per = full >> 3;
        lin = (lin & 7) * per + (lin >> 3);
    }
    const int tm = lin / p.tiles_n;
    const int tn = lin - tm * p.tiles_n;
    const int n0 = tn * BN;
    const int per_img = d.tiles_h * d.tiles_w;
    const int img = tm / per_img;
    const int tr = tm - img * per_img;
    const int th = tr / d.tiles_w;
    const int oh0 = th * 8, ow0 = (tr - th * d.tiles_w) * 8;

    const int N = p.N, K = p.K;
    const int H = d.H, W = d.W, C = d.C;
    const int nk = (K + BK - 1) / BK;
    const int q = tid & 7;
    const int kq = q * 4;
    const int ih0 = oh0 * S - d.PT, iw0 = ow0 * S - d.PL;

    // DMA lanes: quad e = 64 i + lane of the patch is pixel e >> 3 (row-major over the patch),
    // channel quad e & 7; its byte offset without the stage's k (OOB outside the image)
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)d.x, (short)0, (int)d.x_bytes, 0x00020000);
    constexpr unsigned OOB = 0x80000000u;
    // (all byte offsets fit in 31 bits: the launcher checks the extents)
    const unsigned img_off = (unsigned)img * (unsigned)(H * W);
    unsigned poff[PIW];
#pragma unroll
    for (int j = 0; j < PIW; ++j) {
        const int e = (j * 4 + wave) * 64 + lane;
        const int pp = e >> 3;
        const int pr = pp / PWID, pc = pp - (pp / PWID) * PWID;
        const int ih = ih0 + pr, iw = iw0 + pc;
        poff[j] = e < PQUADS && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W
                      ? ((img_off + (unsigned)(ih * W + iw)) * (unsigned)C + (unsigned)kq) * 4u
                      : OOB;
    }
    auto issue_patch = [&](int kt, int buf) __attribute__((always_inline)) {
        const int k0 = kt * BK;
        const bool kok = k0 + kq < K;  // lane & 7 == tid & 7: the DMA lane's channel quad is kq
        float *dst = Ps + buf * PFLOATS;
#pragma unroll
        for (int j = 0; j < PIW; ++j) {
            const int i = j * 4 + wave;
            if (i < PINS) dma16_buf(rx, kok && poff[j] != OOB ? poff[j] + (unsigned)k0 * 4u : OOB, dst + i * 256);
        }
    };

    // depthwise weights [9][C], bias [C] and B through buffer resources: out-of-range quads
    // (k >= K, n >= N, no bias) read as zeros; tap t's weights sit t C floats further (a scalar
    // offset, so the nine loads share one address)
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)d.w, (short)0, 9 * C * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rbias =
        __builtin_amdgcn_make_buffer_rsrc((void *)(d.bias ? d.bias : d.w), (short)0, d.bias ? C * 4 : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rbm = __builtin_amdgcn_make_buffer_rsrc((void *)p.b.p, (short)0, (int)p.b_bytes, 0x00020000);
    unsigned boff[BV];
#pragma unroll
    for (int r = 0; r < BV; ++r) {
        const int n = n0 + (tid >> 3) + 32 * r;
        boff[r] = n < N ? ((unsigned)n * (unsigned)p.b.cs + (unsigned)kq) * 4u : OOB;
    }
    f4 wq[9], bq, breg[BV];
    auto load_regs = [&](int kt) __attribute__((always_inline)) {
        const int k0 = kt * BK;
        const bool kok = k0 + kq < K;
        const unsigned voff = kok ? (unsigned)(k0 + kq) * 4u : OOB;
#pragma unroll
        for (int t = 0; t < 9; ++t)
            wq[t] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rw, voff, t * C * 4, 0));
        bq = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rbias, voff, 0, 0));
#pragma unroll
        for (int r = 0; r < BV; ++r)
            breg[r] = __builtin_bit_cast(
                f4, __builtin_amdgcn_raw_buffer_load_b128(rbm, kok && boff[r] != OOB ? boff[r] + (unsigned)k0 * 4u : OOB, 0, 0));
    };
    // depthwise outputs of this thread's two tile rows from patch buffer buf, into the A tile;
    // the stage's B quads into the B tile
    auto stage_tiles = [&](int buf) __attribute__((always_inline)) {
        const float *ps = Ps + buf * PFLOATS;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int row = (tid >> 3) + 32 * h;
            const int r = row >> 3, c = row & 7;
            f4 v = bq;
#pragma unroll
            for (int i = 0; i < 3; ++i)
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const f4 xv = *reinterpret_cast<const f4 *>(&ps[((r * S + i) * PWID + c * S + j) * 32 + kq]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = fmaf(xv[e], wq[i * 3 + j][e], v[e]);
                }
            *reinterpret_cast<f4 *>(&As[row * LDK + ((q ^ swz(row)) << 2)]) = act4(v, d.act, d.lo, d.hi);
        }
#pragma unroll
        for (int r = 0; r < BV; ++r) {
            const int row = (tid >> 3) + 32 * r;
            *reinterpret_cast<f4 *>(&Bs[row * LDK + ((q ^ swz(row)) << 2)]) = breg[r];
        }
    };

    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    const int li = lane & 31;
    const int lh = lane >> 5;
    const int sw = swz(li);  // fragment rows start at multiples of 32

    if (nk > 0) {
        issue_patch(0, 0);
        load_regs(0);
    }
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = PBUF == 2 ? (kt & 1) : 0;
        wait_vmcnt<0>();
        barrier_lds();  // the stage's patch is in LDS; the A and B tiles are free
        if (PBUF == 2 && kt + 1 < nk) issue_patch(kt + 1, buf ^ 1);
        stage_tiles(buf);
        if (kt + 1 < nk) load_regs(kt + 1);
        barrier_lds();  // A and B tiles complete; the patch is free
        if (PBUF == 1 && kt + 1 < nk) issue_patch(kt + 1, 0);
        if constexpr (BN == 64) {
            f4 af[4], bf[4];
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                af[s2] = *reinterpret_cast<const f4 *>(&As[(wm * 32 + li) * LDK + (((lh * 4 + s2) ^ sw) << 2)]);
                bf[s2] = *reinterpret_cast<const f4 *>(&Bs[(wn * 32 + li) * LDK + (((lh * 4 + s2) ^ sw) << 2)]);
            }
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s2][e], bf[s2][e], acc, 0, 0, 0);
        } else {
            f4 af[2], bf[2];
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                af[s2] = *reinterpret_cast<const f4 *>(&As[(wm * 32 + li) * LDK + (((khalf * 4 + lh * 2 + s2) ^ sw) << 2)]);
                bf[s2] = *reinterpret_cast<const f4 *>(&Bs[li * LDK + (((khalf * 4 + lh * 2 + s2) ^ sw) << 2)]);
            }
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s2][e], bf[s2][e], acc, 0, 0, 0);
        }
    }
    __syncthreads();

    // accumulators -> LDS tile [row][BN] (register r of lane (li, lh): row 8 (r / 4) + 4 lh + r % 4
    // of the wave's 32-row block, column li of its 32-column block)
    float *const Cs = smem;
    if constexpr (BN == 64) {
#pragma unroll
        for (int r = 0; r < 16; ++r) Cs[(wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3)) * LDC + wn * 32 + li] = acc[r];
    } else {
        float *const part = smem + BM * LDC;  // the k 16-31 halves of both row blocks
        if (khalf == 1) {
#pragma unroll
            for (int r = 0; r < 16; ++r) part[wm * 1024 + r * 64 + lane] = acc[r];
        }
        __syncthreads();
        if (khalf == 0) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                Cs[(wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3)) * LDC + li] = acc[r] + part[wm * 1024 + r * 64 + lane];
        }
    }
    __syncthreads();

    // LDS tile -> epilogue -> memory: thread t owns 16-byte column chunk t % (BN / 4) and the
    // tile rows t / (BN / 4) + RSTEP i
    constexpr int C4 = BN / 4;
    constexpr int RSTEP = 256 / C4;
    constexpr int ITERS = BM / RSTEP;
    const float alpha = p.alpha, beta = p.beta, lo = p.lo, hi = p.hi;
    const int act = p.act, OH = d.OH, OW = d.OW;
    const int cl = (tid % C4) * 4;
    const int col = n0 + cl;
    const int r0 = tid / C4;
    if (col >= N) return;
    const int ncol = min(4, N - col);
    const bool full4 = p.vec_out && ncol == 4;
    f4 cbias = {0.f, 0.f, 0.f, 0.f};
    if (p.bias) {
        if (full4) {
            cbias = ldg4(p.bias + col);
        } else {
            for (int e = 0; e < ncol; ++e) cbias[e] = ldg(p.bias + col + e);
        }
    }
    float *const cbase = p.c;
    const float *const rbase = p.res;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int rl = r0 + RSTEP * it;
        const int oh = oh0 + (rl >> 3), ow = ow0 + (rl & 7);
        if (oh >= OH || ow >= OW) continue;
        const long m = ((long)img * OH + oh) * OW + ow;
        f4 v = *reinterpret_cast<const f4 *>(&Cs[rl * LDC + cl]);
        v = v * alpha + cbias;
        if (rbase) {
            const float *src = rbase + m * p.ldr + col;
            if (full4) {
                v += beta * ldg4(src);
            } else {
                for (int e = 0; e < ncol; ++e) v[e] += beta * ldg(src + e);
            }
        }
        v = act4(v, act, lo, hi);
        float *dst = cbase + m * p.ldc + col;
        if (full4) {
            *reinterpret_cast<f4 *>(dst) = v;
        } else {
            for (int e = 0; e < ncol; ++e) dst[e] = v[e];
        }
    }
}

// A whole inverted-residual block (MobileNetV2 with expansion t > 1) as one launch
// (mgc_hip_mbconv): the 1 x 1 expansion of the block input x, its activation, the 3 x 3
// depthwise convolution and its activation are evaluated while the projection GEMM's A operand
// is formed, so neither the expanded tensor (t times the input's channels) nor the depthwise
// output ever goes to memory; the projection's bias, residual and activation are the GEMM's
// epilogue. The reference's C backend runs the three convolutions as three calls with both
// intermediates in its arena (mgc_gemm, mgc_depthwise_nhwc, mgc_gemm: codegen/c.py:1102-1226,
// mgc_kernels.c:370-396, 455-473).
struct MbDev {
    const float *x;   // block input NHWC [n][H][W][Cin]
    const float *we;  // expansion weights packed [Cexp][Cin]
    const float *be;  // expansion bias [Cexp] or null
    const float *wd;  // depthwise weights [9][Cexp]
    const float *bd;  // depthwise bias [Cexp] or null
    int H, W, Cexp, PT, PL, OH, OW;
    float lo_e, hi_e, lo_d, hi_d;  // both activations as clamps: relu [0, inf), clip [lo, hi]
    int tiles_h, tiles_w;  // 8 x 8 output-pixel tiles per image
    long x_bytes;          // bytes of x reachable from d.x (of img for a stem block)
    // stem blocks only: the block input is the 3 x 3, 3-channel stem convolution of img, read
    // through element strides (image, channel, row, column)
    const float *img;
    int iH, iW, iSH, iSW, iPT, iPL;
    unsigned isn, isc, ish, isw;
};

constexpr int kMbMaxCexp = 256;
constexpr int kStemC = 3, kStemK = 3;  // the stem convolution a stem block evaluates: 3 x 3 over 3 channels

// One workgroup (256 threads, four waves) computes an 8 x 8 block of output pixels of one image
// times all N <= 32 projection channels; K runs over the Cexp expanded channels in stages of 32.
//  * The input patch the block's depthwise windows cover ((7 S + 3)^2 pixels x Cin channels) is
//    read once per tile straight into registers as the expansion's B operand: patch pixel block
//    rb (32 pixels) belongs to wave rb % 4, lane (li, h) holding pixel 32 rb + li, input channels
//    h Cin / 2 .. (h + 1) Cin / 2 (the k order the 32 x 32 x 2 MFMA sums over is permuted the
//    same way on both operands).
//  * Per stage each wave multiplies the stage's 32 expansion-weight rows (A) by its pixel blocks
//    (Cin / 2 MFMAs per block), so lane (li, h) ends with pixel li's channels 8 a + 4 h .. + 3
//    (a < 4) of the stage: four quads it biases, clamps (relu or clip as one clamp: fmaxf maps
//    NaN to the lower bound as relu's v > 0 ? v : 0 does), zeroes when the pixel lies outside the
//    image (the depthwise convolution pads the expanded tensor with zeros) and writes to LDS as
//    16-byte stores ([pixel][32] floats, quads XOR-permuted by the pixel so the depthwise reads
//    of eight neighbouring pixels hit different banks). Stride 1 double-buffers the patch (one
//    barrier per stage), stride 2 does not (two barriers; 37 KB per patch).
//  * Lane (li, h) of wave (wm, kh) then computes the depthwise outputs of tile pixel 32 wm + li
//    for the eight stage channels 16 kh + 8 h .. + 7 (nine taps of two 16-byte LDS reads, the
//    depthwise weights and bias of every stage held in LDS for the whole tile) and feeds them
//    straight into the projection MFMAs as their A operand: those are exactly the eight k the
//    lane supplies for rows 32 wm .. 32 wm + 31, with the projection weights B[li][k] in
//    registers (loaded a stage ahead). Biases and depthwise weights sit in LDS for the tile. Waves kh = 0 and 1 sum the two k halves through LDS at
//    the end; the epilogue is the GEMM's.
//  * STEM: the block input is itself a convolution's output, never stored: MobileNetV2's stem
//    (3 x 3 over the 3-channel image, strided, with its activation) ahead of its first block
//    (depthwise and projection, no expansion). The "expansion" is then the stem: lane (li, h)
//    gathers window values k = 16 h .. 16 h + 15 (tap k / 3, channel k % 3; k < 27) of its patch
//    pixel's stem window straight from the image (four-byte loads through element strides, so
//    an NCHW image is read in place), zeros outside the image and for k >= 27, and the weights
//    are the stem's, [Cexp][32] with columns 27..31 zero. The rest is the block as above.
// At least four waves per SIMD: the stride-1 forms fit 128 registers without spilling (four
// workgroups per CU, as their LDS allows); the compiler leaves the stride-2 forms as they are.
template <int S, int KH2, bool STEM>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) mbconv_kernel(const GemmDev p, const MbDev d) {
    static_assert(!STEM || KH2 == 16, "a stem block's window values, 27 padded to 32, are the k operand");
    constexpr int CIN = 2 * KH2;
    constexpr int Q = KH2 / 4;                         // 16-byte quads per lane and row block
    constexpr int PW = 7 * S + 3;                      // patch rows and columns
    constexpr int P = PW * PW;                         // patch pixels
    constexpr int RB = (P + 31) / 32;                  // 32-pixel row blocks of the patch
    constexpr int RBW = (RB + 3) / 4;                  // row blocks per wave (at most)
    constexpr int EBUF = S == 1 ? 2 : 1;
    constexpr int EFLOATS = P * 32;
    constexpr int LDC = 40;
    constexpr int SMEM_LOOP = EBUF * EFLOATS;
    constexpr int SMEM_EPI = 64 * LDC + 2 * 1024;
    constexpr int SMEM_E = SMEM_LOOP > SMEM_EPI ? SMEM_LOOP : SMEM_EPI;
    constexpr int WDF = 11 * kMbMaxCexp;               // depthwise weights [9][256], their bias, expansion bias
    static_assert(S == 1 || S == 2, "stride");
    static_assert(KH2 % 4 == 0, "Cin a multiple of 8");
    __shared__ __attribute__((aligned(16))) float smem[SMEM_E + WDF];
    float *const Wd = smem + SMEM_E;
    // pixel-dependent quad permutation: distinct over 8 consecutive pixels and over 8 pixels at
    // stride 2
    auto fsw = [](int r) __attribute__((always_inline)) { return ((r >> 1) ^ r) & 7; };

    const int tid = threadIdx.x;
    const int lane = tid & 63, li = lane & 31, lh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, kh = wave >> 1;

    // tile order: XCD-aware (consecutive tiles of an image share input rows in one L2)
    const int nb = gridDim.x;
    const int full = nb & ~7;
    int lin = blockIdx.x;
    if (lin < full) {
        const int per = full >> 3;
        lin = (lin & 7) * per + (lin >> 3);
    }
    const int per_img = d.tiles_h * d.tiles_w;
    const int img = lin / per_img;
    const int tr = lin - img * per_img;
    const int th = tr / d.tiles_w;
    const int oh0 = th * 8, ow0 = (tr - th * d.tiles_w) * 8;
    const int ih0 = oh0 * S - d.PT, iw0 = ow0 * S - d.PL;
    const int H = d.H, W = d.W, Cexp = d.Cexp, N = p.N;
    const int nk = (Cexp + 31) / 32;
    constexpr unsigned OOB = 0x80000000u;

    // the expansion's B operand for this wave's patch pixel blocks, and which of the lane's
    // pixels lie inside the image
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void *)(STEM ? d.img : d.x), (short)0, (int)d.x_bytes, 0x00020000);
    f4 xa[RBW][Q];
    unsigned inside = 0;  // bit j: the lane's pixel of row block j is a patch pixel inside the image
    // STEM: the image window every stem output of the patch reads, requested here (coalesced:
    // consecutive threads read consecutive columns of a row of one channel), staged through LDS
    // after the weights' loads and read from there per lane. Rows and columns RW = 2 PW + 1
    // cover the patch's windows at stem strides up to 2; zeros outside the image.
    constexpr int RW = 2 * PW + 1;
    constexpr int RF = kStemC * RW * RW;
    constexpr int RPT = STEM ? (RF + 255) / 256 : 1;
    static_assert(!STEM || RF <= SMEM_E, "the staged window fits the patch buffers");
    float rv[RPT];
    if constexpr (STEM) {
        const int wy0 = ih0 * d.iSH - d.iPT, wx0 = iw0 * d.iSW - d.iPL;  // window origin in the image
        const unsigned ibase = (unsigned)img * d.isn;
#pragma unroll
        for (int u = 0; u < RPT; ++u) {
            const int e = tid + 256 * u;
            const int c = e / (RW * RW), rem = e - c * (RW * RW);
            const int r = rem / RW, col = rem - r * RW;
            const int y = wy0 + r, x = wx0 + col;
            const bool in = e < RF && (unsigned)y < (unsigned)d.iH && (unsigned)x < (unsigned)d.iW;
            const unsigned off =
                in ? (ibase + (unsigned)c * d.isc + (unsigned)y * d.ish + (unsigned)x * d.isw) * 4u : OOB;
            rv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, off, 0, 0));
        }
    }
#pragma unroll
    for (int j = 0; j < RBW; ++j) {
        const int rb = wave + 4 * j;
        const int pa = rb * 32 + li;
        const int pr = pa / PW, pc = pa - (pa / PW) * PW;
        const int ih = ih0 + pr, iw = iw0 + pc;
        const bool ok = rb < RB && pa < P && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
        if constexpr (!STEM) {
            const unsigned base = ((((unsigned)img * (unsigned)H + (unsigned)ih) * (unsigned)W + (unsigned)iw) * CIN +
                                   (unsigned)(lh * KH2)) * 4u;
#pragma unroll
            for (int q = 0; q < Q; ++q)
                xa[j][q] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? base + 16u * q : OOB, 0, 0));
        }
        inside |= (ok ? 1u : 0u) << j;
    }

    // per-stage operands: expansion weight column kt 32 + li (the lane's k half) and its bias;
    // projection weights B[li][kt 32 + 16 kh + 8 lh .. + 7]
    const __amdgpu_buffer_rsrc_t rwe = __builtin_amdgcn_make_buffer_rsrc((void *)d.we, (short)0, Cexp * CIN * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rpb = __builtin_amdgcn_make_buffer_rsrc((void *)p.b.p, (short)0, (int)p.b_bytes, 0x00020000);
    auto load_we = [&](int kt, f4 (&w)[Q]) __attribute__((always_inline)) {
        const int c = kt * 32 + li;
        const bool ok = c < Cexp;
#pragma unroll
        for (int q = 0; q < Q; ++q)
            w[q] = __builtin_bit_cast(
                f4, __builtin_amdgcn_raw_buffer_load_b128(rwe, ok ? ((unsigned)c * CIN + lh * KH2 + 4 * q) * 4u : OOB, 0, 0));
    };
    auto load_pb = [&](int kt, f4 (&b)[2]) __attribute__((always_inline)) {
        const int k0 = kt * 32 + kh * 16 + lh * 8;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = k0 + 4 * h;
            const bool ok = li < N && k < p.K;
            b[h] = __builtin_bit_cast(
                f4, __builtin_amdgcn_raw_buffer_load_b128(rpb, ok ? ((unsigned)li * (unsigned)p.b.cs + k) * 4u : OOB, 0, 0));
        }
    };

    f4 we[Q], pb[2];
    load_we(0, we);
    load_pb(0, pb);
    // depthwise weights, depthwise bias and expansion bias of the channels the stages read into
    // LDS (zeros past Cexp)
    const int cq = nk * 8;  // channel quads of the nk stages
    for (int e = tid; e < 11 * cq; e += 256) {
        const int t = e / cq, c = (e - t * cq) * 4;
        f4 v = {0.f, 0.f, 0.f, 0.f};
        if (c < Cexp) {
            if (t < 9)
                v = ldg4(d.wd + t * Cexp + c);
            else if (t == 9 && d.bd)
                v = ldg4(d.bd + c);
            else if (t == 10 && d.be)
                v = ldg4(d.be + c);
        }
        *reinterpret_cast<f4 *>(&Wd[t * kMbMaxCexp + c]) = v;
    }
    if constexpr (STEM) {
        // the window into LDS (over the patch buffers, which nothing has written yet), then
        // lane (li, h)'s window values k = 16 h .. 16 h + 15 of its patch pixels: tap (ty, tx)
        // and channel c of k are compile-time for either lane half
#pragma unroll
        for (int u = 0; u < RPT; ++u) {
            const int e = tid + 256 * u;
            if (e < RF) smem[e] = rv[u];
        }
        barrier_lds();
#pragma unroll
        for (int j = 0; j < RBW; ++j) {
            const int pa = (wave + 4 * j) * 32 + li;
            const int pr = pa / PW, pc = pa - (pa / PW) * PW;
            const bool ok = (inside >> j) & 1u;
#pragma unroll
            for (int i = 0; i < KH2; ++i) {
                constexpr int kTaps = kStemK * kStemK * kStemC;
                const int k0 = i, k1 = KH2 + i;
                const int t0 = k0 / kStemC, t1 = k1 / kStemC;
                const int ty = lh ? t1 / kStemK : t0 / kStemK;
                const int tx = lh ? t1 % kStemK : t0 % kStemK;
                const int c = lh ? k1 % kStemC : k0 % kStemC;
                const bool kin = lh ? k1 < kTaps : k0 < kTaps;
                // pr, pc < PW and strides <= 2 keep the row and column below RW
                const int idx = ok && kin ? c * (RW * RW) + (pr * d.iSH + ty) * RW + pc * d.iSW + tx : 0;
                const float v = smem[idx];
                xa[j][i >> 2][i & 3] = ok && kin ? v : 0.0f;
            }
        }
        barrier_lds();  // every lane has its window values before the patch buffers are written
    }
    // patch pixels outside the image (or past the patch) are zero in every stage: written once
    // into each patch buffer here, never by the stage loop
#pragma unroll
    for (int j = 0; j < RBW; ++j) {
        const int pix = (wave + 4 * j) * 32 + li;
        if (wave + 4 * j < RB && pix < P && !((inside >> j) & 1u)) {
#pragma unroll
            for (int b = 0; b < EBUF; ++b)
#pragma unroll
                for (int a = 0; a < 4; ++a)
                    *reinterpret_cast<f4 *>(&smem[b * EFLOATS + pix * 32 + 16 * lh + 4 * a]) = f4{0.f, 0.f, 0.f, 0.f};
        }
    }
    barrier_lds();  // the biases and depthwise weights are in LDS before the first expansion reads them
    floatx16 pacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) pacc[r] = 0.0f;
    const int px = wm * 32 + li;                 // this lane's tile pixel for the depthwise pass
    const int ppr = px >> 3, ppc = px & 7;
    const int ch = kh * 16 + lh * 8;             // its eight channels within a stage
    const float lo_e = d.lo_e, hi_e = d.hi_e, lo_d = d.lo_d, hi_d = d.hi_d;

    for (int kt = 0; kt < nk; ++kt) {
        float *const E = smem + (EBUF == 2 ? (kt & 1) * EFLOATS : 0);
        if (EBUF == 1 && kt > 0) barrier_lds();  // every wave's depthwise reads of E are done
        // expansion of this wave's patch row blocks into E
#pragma unroll
        for (int j = 0; j < RBW; ++j) {
            const int rb = wave + 4 * j;
            if (rb < RB) {
                // the accumulators start from the bias of the lane's channels 8 a + 4 lh + e
                floatx16 acc;
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const f4 bq = *reinterpret_cast<const f4 *>(&Wd[10 * kMbMaxCexp + kt * 32 + 8 * a + 4 * lh]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[4 * a + e] = bq[e];
                }
#pragma unroll
                for (int i = 0; i < KH2; ++i)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(we[i >> 2][i & 3], xa[j][i >> 2][i & 3], acc, 0, 0, 0);
                const int pix = rb * 32 + li;
                if ((inside >> j) & 1u) {  // in the image (so also in the patch)
                    const int sw = fsw(pix);
#pragma unroll
                    for (int a = 0; a < 4; ++a) {
                        f4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = fminf(fmaxf(acc[4 * a + e], lo_e), hi_e);
                        *reinterpret_cast<f4 *>(&E[pix * 32 + (((2 * a + lh) ^ sw) << 2)]) = v;
                    }
                }
            }
        }
        if (kt + 1 < nk) load_we(kt + 1, we);
        barrier_lds();  // E complete
        // depthwise outputs of pixel px, channels kt 32 + ch .. + 7: the projection's A operand
        const int cg = kt * 32 + ch;
        f4 a0 = *reinterpret_cast<const f4 *>(&Wd[9 * kMbMaxCexp + cg]);
        f4 a1 = *reinterpret_cast<const f4 *>(&Wd[9 * kMbMaxCexp + cg + 4]);
#pragma unroll 1
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const int prow = (ppr * S + i) * PW + ppc * S + j;
                const int sw = fsw(prow);
                const f4 e0 = *reinterpret_cast<const f4 *>(&E[prow * 32 + (((ch >> 2) ^ sw) << 2)]);
                const f4 e1 = *reinterpret_cast<const f4 *>(&E[prow * 32 + ((((ch >> 2) + 1) ^ sw) << 2)]);
                const f4 w0 = *reinterpret_cast<const f4 *>(&Wd[(i * 3 + j) * kMbMaxCexp + cg]);
                const f4 w1 = *reinterpret_cast<const f4 *>(&Wd[(i * 3 + j) * kMbMaxCexp + cg + 4]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a0[e] = fmaf(e0[e], w0[e], a0[e]);
                    a1[e] = fmaf(e1[e], w1[e], a1[e]);
                }
            }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            a0[e] = fminf(fmaxf(a0[e], lo_d), hi_d);
            a1[e] = fminf(fmaxf(a1[e], lo_d), hi_d);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[e], pb[0][e], pacc, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[e], pb[1][e], pacc, 0, 0, 0);
        if (kt + 1 < nk) load_pb(kt + 1, pb);
    }
    __syncthreads();

    // the two k halves -> LDS tile [64][LDC] (register r of lane (li, lh): row 8 (r / 4) + 4 lh
    // + r % 4 of the wave's 32-row block, column li)
    float *const Cs = smem;
    float *const part = smem + 64 * LDC;
    if (kh == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) part[wm * 1024 + r * 64 + lane] = pacc[r];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            Cs[(wm * 32 + (r >> 2) * 8 + lh * 4 + (r & 3)) * LDC + li] = pacc[r] + part[wm * 1024 + r * 64 + lane];
    }
    __syncthreads();

    // LDS tile -> epilogue -> memory: thread t owns 16-byte column chunk t % 8 and tile rows
    // t / 8 and t / 8 + 32
    const float alpha = p.alpha, beta = p.beta, lo = p.lo, hi = p.hi;
    const int act = p.act, OH = d.OH, OW = d.OW;
    const int cl = (tid & 7) * 4;
    const int r0 = tid >> 3;
    if (cl >= N) return;
    const int ncol = min(4, N - cl);
    const bool full4 = p.vec_out && ncol == 4;
    f4 cbias = {0.f, 0.f, 0.f, 0.f};
    if (p.bias) {
        if (full4) {
            cbias = ldg4(p.bias + cl);
        } else {
            for (int e = 0; e < ncol; ++e) cbias[e] = ldg(p.bias + cl + e);
        }
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int rl = r0 + 32 * it;
        const int oh = oh0 + (rl >> 3), ow = ow0 + (rl & 7);
        if (oh >= OH || ow >= OW) continue;
        const long m = ((long)img * OH + oh) * OW + ow;
        f4 v = *reinterpret_cast<const f4 *>(&Cs[rl * LDC + cl]);
        v = v * alpha + cbias;
        if (p.res) {
            const float *src = p.res + m * p.ldr + cl;
            if (full4) {
                v += beta * ldg4(src);
            } else {
                for (int e = 0; e < ncol; ++e) v[e] += beta * ldg(src + e);
            }
        }
        v = act4(v, act, lo, hi);
        float *dst = p.c + m * p.ldc + cl;
        if (full4) {
            *reinterpret_cast<f4 *>(dst) = v;
        } else {
            for (int e = 0; e < ncol; ++e) dst[e] = v[e];
        }
    }
}

// The 1 x 1 expansion of an inverted-residual block together with the 3 x 3 depthwise
// convolution that alone reads it (mgc_hip_expand_dw), for images whose depthwise window (the
// image plus the padding its outputs reach) fits LDS: a workgroup computes one image times 32
// expanded channels, so the expanded tensor never goes to memory and the depthwise windows need
// nothing from other workgroups; the depthwise output is stored for the projection GEMM. The
// reference's C backend runs the two convolutions as two calls with the expanded tensor in its
// arena (mgc_gemm, mgc_depthwise_nhwc: codegen/c.py:1102-1226, mgc_kernels.c:370-396, 455-473).
struct XdDev {
    const float *x;   // block input NHWC [n][H][W][CIN]
    const float *we;  // expansion weights packed [Cexp][CIN]
    const float *be;  // expansion bias [Cexp] or null
    const float *wd;  // depthwise weights [9][Cexp]
    const float *bd;  // depthwise bias [Cexp] or null
    float *out;       // depthwise output NHWC [n][OH][OW][Cexp]
    int H, W, Cexp, PT, PL, OH, OW;
    int HP, WP;       // window rows and columns: (OH - 1) S + 3, (OW - 1) S + 3
    int slices;       // Cexp / 32
    float lo_e, hi_e, lo_d, hi_d;  // both activations as clamps: relu [0, inf), clip [lo, hi]
    long x_bytes;
};

// One workgroup (four waves) per (image, 32-channel slice), in XCD-aware order so the slices of
// an image share its input in one L2.
//  * Expansion on v_mfma_f32_16x16x4f32 with channels as rows and pixels as columns: 16-pixel
//    row block rb of the image (row-major pixels) belongs to wave rb % 4. For 16-channel chunk c
//    lane (li, g) = (lane % 16, lane / 16) supplies we[channel 16 cb + li][16 c + 4 g + s] and
//    x[pixel 16 rb + li][16 c + 4 g + s] as the s-th MFMA's operands (both permute k alike), so
//    register r of channel block cb's accumulator is channel 16 cb + 4 g + r of pixel
//    16 rb + li: a 16-byte quad, biased, clamped and written to LDS as E[window pixel][quad],
//    the quads XOR-permuted by the pixel so neighbouring pixels' reads spread over the banks.
//  * Every global load is requested when the kernel starts: the slice's weights and biases,
//    which the workgroup reads once into LDS (expansion-weight quads XOR-permuted by the row),
//    then the input quads of a wave's first two row blocks (later ones as earlier ones finish),
//    so filling LDS waits for the weights only. Weights held per lane instead (no LDS copy, no
//    barrier before the expansion) made every wave fetch the whole slice's weights and was
//    slower.
//  * Window pixels outside the image are zero (written once, never by the expansion).
//  * Depthwise: thread t computes channel quad t % 8 of output pixels t / 8, t / 8 + 32, ...:
//    the bias plus the nine taps in row-major order from LDS, clamped, stored as 16 bytes;
//    eight threads cover a pixel's 128 contiguous output bytes.
template <int S, int CIN, int RBW, int EPX>
__global__ void __launch_bounds__(256) gemm_expand_dw_kernel(const XdDev d) {
    constexpr int Q = CIN / 16;     // 16-channel chunks of a pixel
    constexpr int KQ = CIN / 4;     // 16-byte quads of a weight row
    constexpr int WEF = 32 * CIN;   // the slice's expansion weights (floats)
    constexpr int SETS = RBW < 2 ? RBW : 2;
    static_assert(CIN % 32 == 0, "weight quads permuted in groups of eight");
    __shared__ __attribute__((aligned(16))) float smem[EPX * 32 + WEF + 11 * 32];
    float *const E = smem;
    float *const WE = smem + EPX * 32;
    float *const WD = WE + WEF;      // [9][32] depthwise weights, [32] depthwise bias, [32] expansion bias
    auto fsw = [](int r) __attribute__((always_inline)) { return ((r >> 1) ^ r) & 7; };

    const int tid = threadIdx.x;
    const int lane = tid & 63, li = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lin = xcd_block();
    const int img = lin / d.slices;
    const int c0 = (lin - img * d.slices) * 32;
    const int H = d.H, W = d.W, P = H * W, Cexp = d.Cexp, HP = d.HP, WP = d.WP;
    const int rbn = (P + 15) / 16;
    constexpr unsigned OOB = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)d.x, (short)0, (int)d.x_bytes, 0x00020000);

    // the slice's depthwise weights and biases (threads < 88), its expansion weights (CIN / 32
    // quads per thread), then the input quads of row blocks wave + 4 j (j < SETS)
    f4 wdv = {0.f, 0.f, 0.f, 0.f};
    if (tid < 88) {
        const int t = tid >> 3, q4 = (tid & 7) * 4;
        if (t < 9)
            wdv = ldg4(d.wd + (long)t * Cexp + c0 + q4);
        else if (t == 9 && d.bd)
            wdv = ldg4(d.bd + c0 + q4);
        else if (t == 10 && d.be)
            wdv = ldg4(d.be + c0 + q4);
    }
    constexpr int WEQ = WEF / 4 / 256;  // expansion-weight quads per thread
    static_assert(WEQ * 256 * 4 == WEF, "weights spread evenly over the threads");
    f4 wev[WEQ];
#pragma unroll
    for (int i = 0; i < WEQ; ++i) {
        const int e = tid + 256 * i;
        const int r = e / KQ, kq = e - r * KQ;
        wev[i] = ldg4(d.we + (long)(c0 + r) * CIN + 4 * kq);
    }
    f4 xv[SETS][Q];
    auto load_x = [&](int j, f4 (&v)[Q]) __attribute__((always_inline)) {
        const int rb = wave + 4 * j;
        const int pix = 16 * rb + li;
        const bool ok = rb < rbn && pix < P;
        const unsigned base = ((unsigned)(img * P + pix) * CIN + 4u * g) * 4u;
#pragma unroll
        for (int c = 0; c < Q; ++c)
            v[c] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? base + 64u * c : OOB, 0, 0));
    };
#pragma unroll
    for (int j = 0; j < SETS; ++j) load_x(j, xv[j]);

    // window pixels outside the image to zero; the weights into LDS (expansion-weight row r at
    // quad position kq ^ (r & 7))
    for (int e = tid; e < HP * WP * 8; e += 256) {
        const int lp = e >> 3;
        const int py = lp / WP, px = lp - (lp / WP) * WP;
        const int ih = py - d.PT, iw = px - d.PL;
        if ((unsigned)ih >= (unsigned)H || (unsigned)iw >= (unsigned)W)
            *reinterpret_cast<f4 *>(&E[lp * 32 + (e & 7) * 4]) = f4{0.f, 0.f, 0.f, 0.f};
    }
    if (tid < 88) *reinterpret_cast<f4 *>(&WD[(tid >> 3) * 32 + (tid & 7) * 4]) = wdv;
#pragma unroll
    for (int i = 0; i < WEQ; ++i) {
        const int e = tid + 256 * i;
        const int r = e / KQ, kq = e - r * KQ;
        *reinterpret_cast<f4 *>(&WE[r * CIN + ((kq ^ (r & 7)) << 2)]) = wev[i];
    }
    barrier_lds();

    // expansion of this wave's row blocks into the window
    const float lo_e = d.lo_e, hi_e = d.hi_e;
    const f4 be0 = *reinterpret_cast<const f4 *>(&WD[320 + 4 * g]);
    const f4 be1 = *reinterpret_cast<const f4 *>(&WD[320 + 16 + 4 * g]);
    const int wrow0 = li * CIN, wrow1 = (16 + li) * CIN, wsw = li & 7;
#pragma unroll
    for (int j = 0; j < RBW; ++j) {
        const int rb = wave + 4 * j;
        if (rb >= rbn) break;
        f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < Q; ++c) {
            const int kq = 4 * c + g;
            const f4 w0 = *reinterpret_cast<const f4 *>(&WE[wrow0 + ((kq ^ wsw) << 2)]);
            const f4 w1 = *reinterpret_cast<const f4 *>(&WE[wrow1 + ((kq ^ wsw) << 2)]);
            const f4 xq = xv[j % SETS][c];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(w0[s], xq[s], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(w1[s], xq[s], acc1, 0, 0, 0);
            }
        }
        if (j + SETS < RBW) load_x(j + SETS, xv[j % SETS]);
        const int pix = 16 * rb + li;
        const int ih = pix / W, iw = pix - (pix / W) * W;
        const int py = ih + d.PT, px = iw + d.PL;
        if (pix < P && py < HP && px < WP) {
            const int lp = py * WP + px, sw = fsw(lp);
            f4 v0, v1;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v0[e] = fminf(fmaxf(acc0[e] + be0[e], lo_e), hi_e);
                v1[e] = fminf(fmaxf(acc1[e] + be1[e], lo_e), hi_e);
            }
            *reinterpret_cast<f4 *>(&E[lp * 32 + ((g ^ sw) << 2)]) = v0;
            *reinterpret_cast<f4 *>(&E[lp * 32 + (((4 + g) ^ sw) << 2)]) = v1;
        }
    }
    barrier_lds();

    // depthwise outputs: channel quad q of pixels tid / 8 + 32 i
    const int q = tid & 7;
    f4 wt[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) wt[t] = *reinterpret_cast<const f4 *>(&WD[t * 32 + 4 * q]);
    const f4 bd = *reinterpret_cast<const f4 *>(&WD[288 + 4 * q]);
    const float lo_d = d.lo_d, hi_d = d.hi_d;
    const int OH = d.OH, OW = d.OW, OP = OH * OW;
    float *const obase = d.out + (long)img * OP * Cexp + c0 + 4 * q;
    for (int op = tid >> 3; op < OP; op += 32) {
        const int oh = op / OW, ow = op - (op / OW) * OW;
        f4 a = bd;
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const int lp = (oh * S + i) * WP + ow * S + j;
                const f4 e = *reinterpret_cast<const f4 *>(&E[lp * 32 + ((q ^ fsw(lp)) << 2)]);
#pragma unroll
                for (int k = 0; k < 4; ++k) a[k] = fmaf(e[k], wt[3 * i + j][k], a[k]);
            }
#pragma unroll
        for (int k = 0; k < 4; ++k) a[k] = fminf(fmaxf(a[k], lo_d), hi_d);
        *reinterpret_cast<f4 *>(obase + (long)op * Cexp) = a;
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

// Sum of the K-split partials src[0], src[stride], ..., src[(split - 1) * stride] in split
// order; the loads of up to four splits go out together, so a reduction waits for one or two
// memory round trips instead of one per split.
__device__ __forceinline__ f4 sum_partials(const f4 *src, long stride, int split) {
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
    f4 v = src[0];
    for (int s0 = 1; s0 < split; s0 += 4) {
        f4 part[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) part[u] = s0 + u < split ? src[(long)(s0 + u) * stride] : zero4;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (s0 + u < split) v += part[u];
    }
    return v;
}

// The same for N % 4 == 0 with 16-byte aligned output rows: four columns per thread, 16-byte
// partial loads and stores (element sums in the same split order as above). The bias and
// residual chunks are requested before the partials, so their loads overlap.
__global__ void gemm_splitk_reduce_vec4(const GemmDev p, FastDiv div_n4) {
    const int N4 = p.N >> 2;
    const int total4 = p.M * N4;
    const long stride4 = ((long)p.M * p.N) >> 2;
    const f4 *ws4 = reinterpret_cast<const f4 *>(p.ws);
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const int bmode = p.bias ? p.bias_mode : 0;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total4; idx += gridDim.x * blockDim.x) {
        const int row = fdiv(idx, div_n4);
        const int col = (idx - row * N4) * 4;
        const f4 bcol = bmode == 1 ? ldg4(p.bias + col) : zero4;
        const float brow = bmode == 2 ? ldg(p.bias + row) : 0.0f;
        const f4 rv = p.res ? ldg4(p.res + (long)row * p.ldr + col) : zero4;
        f4 v = sum_partials(ws4 + idx, stride4, p.split);
        v = v * p.alpha;
        if (bmode == 2) v += brow;
        if (bmode == 1) v += bcol;
        if (p.res) v += p.beta * rv;
        *reinterpret_cast<f4 *>(p.c + (long)row * p.ldc + col) = act4(v, p.act, p.lo, p.hi);
    }
}

// The same reduction for a GEMM whose output feeds a LayerNorm over its rows (N % 4 == 0,
// N <= 1024): one wavefront per row sums the partials, applies the epilogue exactly as
// gemm_splitk_reduce_vec4 does, stores the GEMM output when p.c is set (other readers need it)
// and normalizes the row from registers (layer_norm_row_vec4, as the LayerNorm kernel does), so
// the row makes no second trip through HBM and the LayerNorm needs no launch of its own. Every
// load the row needs (partials, bias, residual, the LayerNorm's scale and bias) is requested
// before the first is used.
__global__ void __launch_bounds__(256) gemm_splitk_layer_norm(const GemmDev p, const float4 *ln_scale,
                                                              const float4 *ln_bias, float eps, float4 *ln_out) {
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (row >= p.M) return;
    const int N4 = p.N >> 2;
    const long total4 = ((long)p.M * p.N) >> 2;
    const f4 *ws4 = reinterpret_cast<const f4 *>(p.ws) + (long)row * N4;
    const f4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const int bmode = p.bias ? p.bias_mode : 0;
    f4 bcol[4], rv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = lane + 64 * j;
        const int col = k * 4;
        const bool ok = k < N4;
        bcol[j] = ok && bmode == 1 ? ldg4(p.bias + col) : zero4;
        rv[j] = ok && p.res ? ldg4(p.res + (long)row * p.ldr + col) : zero4;
    }
    const float brow = bmode == 2 ? ldg(p.bias + row) : 0.0f;
    const LnAffine aff = ln_affine_load(lane, N4, ln_scale, ln_bias);
    // partials summed in split order, as gemm_splitk_reduce_vec4 does
    f4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = lane + 64 * j;
        acc[j] = k < N4 ? ws4[k] : zero4;
    }
    for (int s0 = 1; s0 < p.split; s0 += 4) {
        f4 part[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = lane + 64 * j;
                part[u][j] = s0 + u < p.split && k < N4 ? ws4[(long)(s0 + u) * total4 + k] : zero4;
            }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (s0 + u < p.split) {
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[j] += part[u][j];
            }
    }
    float4 y[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = lane + 64 * j;
        y[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (k < N4) {
            const int col = k * 4;
            f4 v = acc[j] * p.alpha;
            if (bmode == 2) v += brow;
            if (bmode == 1) v += bcol[j];
            if (p.res) v += p.beta * rv[j];
            v = act4(v, p.act, p.lo, p.hi);
            if (p.c) *reinterpret_cast<f4 *>(p.c + (long)row * p.ldc + col) = v;
            y[j] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
    layer_norm_row_vec4(y, lane, N4, aff, eps, ln_out + (long)row * N4);
}

static bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15) == 0; }

static bool bs_div4(const long *bs, int rank) {
    for (int d = 0; d < rank; ++d)
        if (bs[d] % 4) return false;
    return true;
}

typedef void (*GemmKernel)(const GemmDev);
typedef void (*GemmKernelStream)(const GemmDev, int, int, int, float, float, long, long);

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

template <int BM, int BN, int WGM>
static GemmKernel pick_dma(int am) {
    return am == AM_VEC   ? &gemm_dma_kernel<BM, BN, WGM, 2, AM_VEC>
           : am == AM_CAT ? &gemm_dma_kernel<BM, BN, WGM, 2, AM_CAT>
                          : &gemm_dma_kernel<BM, BN, WGM, 2, AM_CONV_VEC>;
}

static GemmKernel pick_dma_tail(int am) {
    return am == AM_VEC   ? &gemm_dma_tail_kernel<AM_VEC>
           : am == AM_CAT ? &gemm_dma_tail_kernel<AM_CAT>
                          : &gemm_dma_tail_kernel<AM_CONV_VEC>;
}

// 16 x 16 wave-split launches: eight waves with three-stage rings for K of 1024 and more (two
// waves per SIMD, one computing while the other waits for its loads), four waves with
// two-stage rings below. Measured against each other (same table as use_tile16): eight waves
// 5.9 / 7.3 / 6.7 us on 196 x 256 x 1024 / 49 x 512 x 2048 / 1 x 1000 x 2048 against 6.2 /
// 8.2 / 7.9 with four waves and four stages; four waves 5.6 us on 784 x 128 x 512 against 7.1
// with eight; rings of 6 and 8 stages were slower throughout.
static int wsplit16_waves(int K) { return K >= 1024 ? 8 : 4; }

template <int STAGES, int WAVES>
static GemmKernel pick16(int am) {
    return am == AM_VEC   ? &gemm_dma_wsplit16_kernel<AM_VEC, STAGES, WAVES>
           : am == AM_CAT ? &gemm_dma_wsplit16_kernel<AM_CAT, STAGES, WAVES>
                          : &gemm_dma_wsplit16_kernel<AM_CONV_VEC, STAGES, WAVES>;
}

static GemmKernel pick_wsplit16(int am, int K) { return wsplit16_waves(K) == 8 ? pick16<3, 8>(am) : pick16<2, 4>(am); }

static GemmKernel pick_wsplit(int am) {
    return am == AM_VEC   ? &gemm_dma_wsplit_kernel<AM_VEC>
           : am == AM_CAT ? &gemm_dma_wsplit_kernel<AM_CAT>
                          : &gemm_dma_wsplit_kernel<AM_CONV_VEC>;
}

struct TileChoice {
    int bm, bn, split;
};

static const int kCUs = 256;

// Tile shape and K split for one GEMM. 64 x 64 tiles throughout: a two-stage ring is 32 KB of
// LDS and the hardware runs four such workgroups per CU (the occupancy query says five), whose
// interleaved waves hide each other's load latency. Measured on every ResNet-50 b32 GEMM this
// beats 128 x 64 and 128 x 128 tiles (which fit one or two workgroups per CU) and persistent
// tile-streaming kernels.
//
// K is split over extra workgroups when the tiles alone leave CUs idle or badly balanced:
// with W workgroups on the 256 CUs the busiest CU runs ceil(W / 256) of them while the
// average is W / 256, so the split is raised until that ratio reaches 0.9 (at most 5 * 256
// workgroups, at least 256 k per split). Balancing alone pays only for long K (>= 2048): the
// partial results cost a write and a read of split * M * N floats. The cap of 5 * 256 is
// measured: the 14 x 14 3 x 3 convolutions of ResNet-50 b32 (392 tiles, K 2304) split in three
// (1176 workgroups) take 81 us, capped at 4 * 256 (no split) 89 us.
static TileChoice choose_tiles(int M, int N, int K, int batch) {
    TileChoice t;
    t.bm = 64;
    t.bn = 64;
    t.split = 1;
    const long tiles = (long)((M + 63) / 64) * ((N + 63) / 64) * batch;
    if (batch != 1 || K < 512 || !(tiles < kCUs || (K >= 2048 && tiles < 2 * kCUs))) return t;
    auto balance = [&](int s) {
        const long w = tiles * s;
        return (double)w / (double)(((w + kCUs - 1) / kCUs) * kCUs);
    };
    const int max_split = K / 256 < 8 ? K / 256 : 8;
    double best = balance(1);
    for (int s = 2; s <= max_split && tiles * s <= 5L * kCUs && best < 0.9; ++s) {
        const double e = balance(s);
        if (e > best + 0.05) {
            best = e;
            t.split = s;
        }
    }
    // too few tiles to fill the chip even once: split further, as far as K allows without
    // spilling into a second round (tiles * split <= kCUs), where the CUs that run two
    // workgroups would double the time
    if (tiles * t.split < kCUs) {
        const int fill = (int)(kCUs / tiles);
        const int s = fill < max_split ? fill : max_split;
        if (s > t.split) t.split = s;
    }
    return t;
}

// The wave-split kernel (32 x 32 tiles, K dealt to the four waves of a workgroup) in place of
// the 64 x 64 tiles for a GEMM that the latter would split over K: returns the wave-split
// launch's own K split (1: none, so no reduction launch) or 0 to keep the 64 x 64 tiles. Cost
// of a launch = the K stages one wave runs, plus six when a reduction launch follows (about
// what that launch and the partials' round trip cost); the wave-split launch may use up to the
// 64 x 64 launch's split (the workspace is sized for it) while its tiles fit one round of two
// workgroups per CU (its LDS allows two). Ties go to the wave-split kernel, the smaller split.
// Batch-1 convolutions at 56 x 56 and 28 x 28 and the 128-row QKV and FFN GEMMs of a sequence
// take it without a split; deep-K layers on 14 x 14 and 7 x 7 images with one, four times as
// many waves sharing K as the 64 x 64 split launch. Measured at batch 1 with the no-split form
// only, two workgroups per CU against one: BERT-base 0.955 vs 1.113 ms, ResNet-50 and
// MobileNetV2 unchanged; a reduction cost of 2, 8 and 16 stages instead of 4: ResNet-50 0.557,
// 0.561, 0.580 vs 0.556 ms. With the split form as well (ResNet-50 b1 0.511 ms), a reduction
// cost of 4, 8 or 10 stages instead of 6 moves ResNet-50, MobileNetV2 and BERT-base at batch 1
// by less than 0.3%.
static int wave_split(int M, int N, int K, int batch) {
    const TileChoice t = choose_tiles(M, N, K, batch);
    if (batch != 1) return 0;
    const long tiles32 = (long)((M + 31) / 32) * ((N + 31) / 32);
    if (t.split < 2) {
        // K too short to split (< 512) on too few 64 x 64 tiles: four times the tiles with a
        // quarter of the stages per wave, when that is fewer stages (the 1 x 1 convolutions of
        // 28 x 28 and 14 x 14 images at batch 1, MobileNetV2's 14 x 14 projections at batch 32),
        // up to three 32 x 32 tiles per CU (a partial second round of its two workgroups per CU
        // still beats the 128 x 32 tiles' single round: MobileNetV2 b32's 6272 x 96 x 576
        // projections, 588 tiles, 16.2 -> 13.2 us; forward 0.572 -> 0.562 ms)
        const long tiles64 = (long)((M + 63) / 64) * ((N + 63) / 64);
        const int st = (K + 31) / 32;
        return tiles64 < kCUs && tiles32 <= 3 * kCUs && (st + 3) / 4 < st ? 1 : 0;
    }
    auto chunk_stages = [&](int s) { return ((K + s - 1) / s + 31) / 32; };
    constexpr int kReduce = 6;
    int best = 0, best_cost = chunk_stages(t.split) + kReduce;
    for (int s = 1; s <= t.split && tiles32 * s <= 2 * kCUs; ++s) {
        const int cost = (chunk_stages(s) + 3) / 4 + (s > 1 ? kReduce : 0);
        if (cost < best_cost || (best == 0 && cost == best_cost)) {
            best = s;
            best_cost = cost;
        }
    }
    return best;
}

// 16 x 16 tiles instead of the 32 x 32 wave-split launch: when there are at most two of them
// per CU (512) and K is at most 2560. Graph replays of 16 independent GEMMs per shape at batch 1
// on MI355X, us per GEMM, 32 x 32 wave split (with its K split and reduction where it takes
// one) against 16 x 16: 784 x 128 x 512 6.8 / 5.6, 196 x 256 x 1024 9.1 / 5.9, 196 x 512 x 1024
// 9.3 / 7.4, 49 x 2048 x 512 6.9 / 6.2, 49 x 512 x 2048 9.9 / 7.3, 1 x 1000 x 2048 9.0 / 6.7,
// 128 x 768 x 768 8.1 / 6.9; 3 x 3 convolutions 28 x 28 x 128 11.5 / 8.1, 14 x 14 x 256
// 12.7 / 8.9. Where the rule says no: 128 x 2304 x 768 (1152 tiles) 12.0 / 14.4,
// 128 x 3072 x 768 12.3 / 16.8, 196 x 1024 x 256 6.0 / 7.5, 56 x 56 x 64 3 x 3 8.0 / 7.9,
// deep K: 128 x 768 x 3072 14.7 / 15.5, 7 x 7 x 512 3 x 3 (K 4608) 12.9 / 13.0.
// Deeper K (the 3 x 3 convolutions of a 7 x 7 image, K 4608) splits into chunks of at most 2304
// when the split tiles still number at most 512 and the workspace allows the split (wsk, the
// 32 x 32 launch's split, is what it was sized for); returns that split, 1 without, 0 for the
// 32 x 32 tiles.
static int use_tile16(int M, int N, int K, int wsk) {
    const long tiles16 = (long)((M + 15) / 16) * ((N + 15) / 16);
    if (K <= 2560) return tiles16 <= 2 * kCUs ? 1 : 0;
    const int s = (K + 2303) / 2304;
    return s <= wsk && tiles16 * s <= 2 * kCUs ? s : 0;
}

// Quarter tiles for the last tiles of a 64 x 64 launch: with T = q * 256 + r tiles (0 < r <=
// kQuarterTiles, q >= 1) the busiest CUs would run q + 1 tiles while most run q; the last r
// tiles are computed as 4 r quarter tiles instead (a quarter's MFMA work is a fourth), so no
// CU runs more than q tiles and one quarter. For short K a quarter's fixed costs (first
// stage, epilogue) outweigh its share of the work, and with r > 64 CUs would run two or more
// quarters (MobileNetV2 b32 0.693 -> 0.704 ms with r <= 128 at any K; ResNet-50 b32 the same
// within 0.3%; K >= 128 against K >= 256: ResNet-50 b32 2.764 -> 2.759 ms). The quarter form reads 64 k per ring stage: convolution windows need channel
// groups of a multiple of 64, a concatenated K a first part of a multiple of 64.
static const int kQuarterTiles = 64;
static const int kQuarterMinK = 128;
// With K >= 512 a quarter's fixed costs weigh less, and tails of up to 128 tiles run as quarters
// too: BERT-base b16's 1152-tile Q/K/V projection (K 768), forward 3.434 -> 3.381 ms; GPT-2 and
// ResNet-50 have no such launch and are unchanged.
static const int kQuarterTilesDeepK = 128;
// A launch of between one and two tiles per CU (256 < T < 512) without a K split runs its first
// T / 2 tiles whole and the rest as quarters, so the CUs share the second half evenly instead of
// T - 256 of them running a second whole tile: ResNet-50 b32's five 392-tile 1 x 1 layers (K
// 1024) 38.1 -> 35.3 us, forward 2.767 -> 2.753 ms. Deep K only: the quarters' fixed costs
// weigh more where K is short, and launches that split K over workgroups already fill the chip
// (as half whole tiles and half quarters instead of a split and reduction they were slower:
// ResNet-50 b32 2.774 -> 2.950 ms).
static const int kHalfQuarterMinK = 512;

static bool quarter_tiles_ok(int am, const GemmDev &p) {
    return am == AM_VEC || (am == AM_CONV_VEC && p.a.cg % 64 == 0) || (am == AM_CAT && p.k1 % 64 == 0);
}

// The streaming kernel for short K over many rows (K <= 32, K % 4 == 0, at least 4096 rows,
// at most 768 columns).
static bool use_stream(int M, int N, int K) { return K <= 32 && K % 4 == 0 && M >= 4096 && N <= 24 * 32; }
// The same over an NHWC image (one channel group, C % 4 == 0) for K <= 48 and one 32-column
// block, where the tiled kernel spends a whole 128-row tile's prologue and epilogue on two K
// stages: MobileNetV2 b32's stem (401408 x 32 x 48) 33.3 -> 25.0 us, forward 0.562 -> 0.556 ms.
static bool use_stream_conv(int M, int N, int K) { return K <= 48 && K % 4 == 0 && M >= 4096 && N <= 32; }
static bool stream_act(int act) { return act == MGC_ACT_NONE || act == MGC_ACT_RELU || act == MGC_ACT_CLIP; }

template <int KH, bool CONV>
static GemmKernelStream pick_stream(int nb) {
    return nb == 1   ? &gemm_stream_kernel<KH, 1, CONV>
           : nb == 2 ? &gemm_stream_kernel<KH, 2, CONV>
                     : &gemm_stream_kernel<KH, 3, CONV>;
}

// Column groups of at most three 32-column blocks (the B registers of one group), as even as
// the block count allows: wider groups (five and six blocks, one wave per SIMD) were slower
// than the tiled kernel on MobileNetV2's 24 -> 144 and 32 -> 192 layers at batch 32 (27.0 /
// 13.2 us against 23.8 / 11.5), three blocks faster (16 -> 96: 32.1 against 49.5); as many waves as the kernel's registers let the CUs hold at once
// (each wave loops over its tiles, so a second round of waves would only start late).
static void stream_launch(mgc_hip_exec *x, const GemmDev &p) {
    const int blocks = (p.N + 31) / 32;
    const int groups = (blocks + 2) / 3;
    const int nb = (blocks + groups - 1) / groups;
    const int tiles_m = (p.M + 31) / 32;
    const bool conv = p.a.kind == MGC_OP_CONV_NHWC;
    const int kh = p.K <= 16 ? 0 : p.K <= 32 ? 1 : 2;
    const GemmKernelStream kern = conv ? (kh == 0 ? pick_stream<8, true>(nb) : kh == 1 ? pick_stream<16, true>(nb)
                                                                                  : pick_stream<24, true>(nb))
                                       : (kh == 0 ? pick_stream<8, false>(nb) : pick_stream<16, false>(nb));
    static int resident[2][3][4];  // workgroups per CU, by (CONV, KH, NB); 0 = not asked yet
    int &per_cu = resident[conv ? 1 : 0][kh][nb];
    if (per_cu == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(kern), 256, 0) !=
                hipSuccess || n < 1)
            n = 1;
        per_cu = n;
    }
    const int waves = per_cu * 4 * kCUs;
    int per_group = waves / groups;
    if (per_group > tiles_m) per_group = tiles_m;
    if (per_group < 1) per_group = 1;
    const int wgs = (groups * per_group + 3) / 4;
    const int clamp = p.act == MGC_ACT_CLIP || p.act == MGC_ACT_RELU;
    const float lo = p.act == MGC_ACT_CLIP ? p.lo : 0.0f;
    const float hi = p.act == MGC_ACT_CLIP ? p.hi : INFINITY;
    const long c_bytes = ((long)(p.M - 1) * p.ldc + p.N) * 4;
    const long r_bytes = p.res ? ((long)(p.M - 1) * p.ldr + p.N) * 4 : 0;
    MGC_LAUNCH(x, kern, dim3((unsigned)wgs), dim3(256), 0, p, groups, per_group, clamp, lo, hi, c_bytes, r_bytes);
}

// The same choice for a GEMM whose split-K reduction ends in a LayerNorm (the split is
// required, at least 2 and at most the 64 x 64 launch's): the wave-split launch with the split
// that needs the fewest K stages per wave, when that beats the 64 x 64 launch; 0 to keep the
// 64 x 64 tiles. Both end in the same reduction launch, so stages alone decide.
static int wave_split_ln(int M, int N, int K, int split) {
    const long tiles32 = (long)((M + 31) / 32) * ((N + 31) / 32);
    auto chunk_stages = [&](int s) { return ((K + s - 1) / s + 31) / 32; };
    int best = 0, best_cost = chunk_stages(split);
    for (int s = 2; s <= split && tiles32 * s <= 2 * kCUs; ++s) {
        const int cost = (chunk_stages(s) + 3) / 4;
        if (cost < best_cost) {
            best = s;
            best_cost = cost;
        }
    }
    return best;
}

// 128 x 32 tiles (four waves stacked along M) instead of 64 x 64 when they pad N less: the
// pointwise convolutions of MobileNet-style networks have 16 to 160 output channels, where a
// 64-wide tile leaves up to 3/4 of the matrix-core work and of the epilogue on padding. Only
// without a K split (the workspace size depends on the tile count) and for the DMA kernel.
static bool narrow_tiles(int N, int split) {
    const long pad64 = (N + 63) / 64 * 64, pad32 = (N + 31) / 32 * 32;
    return split == 1 && pad32 < pad64;
}

}  // namespace mgc

using namespace mgc;

extern "C" long mgc_hip_gemm_workspace(int M, int N, int K, int batch) {
    TileChoice t = choose_tiles(M, N, K, batch);
    return t.split > 1 ? (long)t.split * M * N : 0;
}

// LayerNorm that ends a split-K GEMM (mgc_hip_gemm_layer_norm).
struct LnTail {
    const float *scale, *bias;
    float eps;
    float *out;
};

// K splits of a GEMM whose reduction ends in a LayerNorm: the library's own choice, and at
// least two, since the reduction is where the LayerNorm runs.
static int ln_split(int M, int N, int K) {
    const TileChoice t = choose_tiles(M, N, K, 1);
    return t.split > 1 ? t.split : 2;
}

static void gemm_launch(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const LnTail *ln);

extern "C" void mgc_hip_gemm(mgc_hip_exec *x, const mgc_hip_gemm_args *g) { gemm_launch(x, g, nullptr); }

// ---------------------------------------------------------------------------------------------
// mgc_hip_gemm_noalloc: mgc_hip_gemm with the K-split partials in the library's own device
// array instead of a caller workspace, for callers that cannot allocate device memory.
//
// `scratch` is a file-scope device array; every GPU the library runs on holds its own copy
// (MGC_HIP_NOALLOC_SCRATCH_FLOATS floats) until the process ends. Host code never passes the
// array's name to a kernel (on the host it is only a stand-in symbol): the first call on a
// device, with that device current, asks the runtime for that device's address of the array
// and keeps it; kernels get that pointer. Every call on a GPU shares its array, so calls that
// overlap on one GPU (different streams, or threads without ordering) race on it; calls on one
// stream are ordered and safe. Nothing in it must start at zero: each K split writes its whole
// partial tile (zeros for an empty K range) before the reduction reads it.
static __device__ __align__(256) float scratch[MGC_HIP_NOALLOC_SCRATCH_FLOATS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch`, looked up once per device (with the device current).
hipError_t scratch_for_current_device(float **out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return err;
        g_scratch_ptr[dev] = static_cast<float *>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}
}  // namespace

extern "C" int mgc_hip_gemm_noalloc(void *stream, const mgc_hip_gemm_args *g) {
    if (!g) {
        set_error("mgc_hip_gemm_noalloc: no arguments", hipErrorInvalidValue);
        return MGC_ERR_ARGS;
    }
    int batch = 1;
    for (int d = 0; d < g->batch_rank && d < 4; ++d) batch *= g->batch_dims[d];
    // A caller's explicit split must fit the scratch. The library's own choice (split_k 0) is
    // taken as mgc_hip_gemm takes it with a workspace of the scratch's size: a split whose
    // partials would not fit is dropped (one K pass, no reduction), never refused. (choose_tiles
    // keeps its partials within 5 * 256 tiles of 64 x 64 floats, 20 MiB, so with this scratch
    // size that does not happen.)
    long need = 0;
    if (g->M > 0 && g->N > 0 && g->K > 0 && batch > 0 && g->split_k > 1 && batch == 1)
        need = (long)g->split_k * g->M * g->N;
    if (need > MGC_HIP_NOALLOC_SCRATCH_FLOATS) {
        char msg[200];
        snprintf(msg, sizeof msg,
                 "mgc_hip_gemm_noalloc: this GEMM needs %ld floats of K-split scratch, more than "
                 "the %ld the library holds",
                 need, (long)MGC_HIP_NOALLOC_SCRATCH_FLOATS);
        set_error(msg, hipErrorInvalidValue);
        return MGC_ERR_ARGS;
    }
    float *ws = nullptr;
    const hipError_t err = scratch_for_current_device(&ws);
    if (err != hipSuccess) {
        set_error("mgc_hip_gemm_noalloc: hipGetSymbolAddress(scratch)", err);
        return MGC_ERR_HIP;
    }
    mgc_hip_gemm_args a = *g;
    a.workspace = ws;
    a.workspace_floats = MGC_HIP_NOALLOC_SCRATCH_FLOATS;
    mgc_hip_exec x{};
    x.stream = static_cast<hipStream_t>(stream);
    // an error the caller left pending on this thread is not this call's: the launch check
    // after each kernel reads hipGetLastError()
    (void)hipGetLastError();
    gemm_launch(&x, &a, nullptr);
    if (!x.launch_error) return MGC_OK;
    // gemm_launch reports operands outside a kernel's limits as hipErrorInvalidValue
    return x.launch_error == (int)hipErrorInvalidValue ? MGC_ERR_ARGS : MGC_ERR_HIP;
}

extern "C" int mgc_hip_gemm_layer_norm_supported(int M, int N) {
    return M >= 1 && M < (1 << 25) && N >= 4 && N % 4 == 0 && N <= 1024;
}

extern "C" long mgc_hip_gemm_layer_norm_workspace(int M, int N, int K) {
    if (!mgc_hip_gemm_layer_norm_supported(M, N) || K < 1) return 0;
    return (long)ln_split(M, N, K) * M * N;
}

extern "C" void mgc_hip_gemm_layer_norm(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const float *ln_scale,
                                        const float *ln_bias, float eps, float *ln_out) {
    if (g->M <= 0) return;
    const int split = ln_split(g->M, g->N, g->K);
    const bool ok = mgc_hip_gemm_layer_norm_supported(g->M, g->N) && g->batch_rank == 0 &&
                    g->workspace != nullptr && g->workspace_floats >= (long)split * g->M * g->N &&
                    aligned16(g->workspace) && aligned16(ln_out) && aligned16(ln_scale) &&
                    aligned16(ln_bias) && (!g->c || (aligned16(g->c) && g->ldc % 4 == 0)) &&
                    (!g->res || (aligned16(g->res) && g->ldr % 4 == 0)) &&
                    (!g->bias || g->bias_mode != 1 || aligned16(g->bias));
    if (!ok) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_gemm_layer_norm: shape, alignment or workspace outside its limits",
                  hipErrorInvalidValue);
        return;
    }
    mgc_hip_gemm_args a = *g;
    a.split_k = split;
    const LnTail tail{ln_scale, ln_bias, eps, ln_out};
    gemm_launch(x, &a, &tail);
}

extern "C" void mgc_hip_gemm_dw(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const mgc_hip_dw_args *dw) {
    if (g->M <= 0 || g->N <= 0) return;
    const long ohw = (long)dw->OH * dw->OW;
    const long n_img = ohw > 0 ? g->M / ohw : 0;
    const long x_bytes = n_img * dw->H * dw->W * (long)dw->C * 4;
    const long b_bytes = ((long)(g->N - 1) * g->b.cs + g->K) * 4;
    const bool ok = g->batch_rank == 0 && g->k1 == 0 && g->K == dw->C && dw->C > 0 && dw->C % 4 == 0 &&
                    dw->H > 0 && dw->W > 0 && dw->SH == dw->SW && (dw->SH == 1 || dw->SH == 2) && ohw > 0 &&
                    g->M % ohw == 0 && x_bytes < 0x7fffffffL && b_bytes < 0x7fffffffL &&
                    9L * dw->C * 4 < 0x7fffffffL && (!g->bias || g->bias_mode == 1) &&
                    g->b.kind == MGC_OP_STRIDED && g->b.rs == 1 && g->b.cs >= g->K && g->b.cs % 4 == 0 &&
                    aligned16(g->b.p) && aligned16(dw->x) && aligned16(dw->w) && aligned16(dw->bias);
    if (!ok) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_gemm_dw: shape, layout or alignment outside its limits", hipErrorInvalidValue);
        return;
    }
    GemmDev p{};
    p.M = g->M;
    p.N = g->N;
    p.K = g->K;
    p.b = g->b;
    p.c = g->c;
    p.ldc = g->ldc;
    p.alpha = g->alpha;
    p.beta = g->beta;
    p.bias = g->bias;
    p.bias_mode = g->bias ? 1 : 0;
    p.res = g->res;
    p.ldr = g->ldr;
    p.act = g->act;
    p.lo = g->lo;
    p.hi = g->hi;
    p.split = 1;
    p.nbatch = 1;
    p.b_bytes = b_bytes;
    p.vec_out = p.ldc % 4 == 0 && aligned16(p.c) && (!p.res || (p.ldr % 4 == 0 && aligned16(p.res))) &&
                aligned16(p.bias);
    DwDev d;
    d.x = dw->x;
    d.w = dw->w;
    d.bias = dw->bias;
    d.H = dw->H;
    d.W = dw->W;
    d.C = dw->C;
    d.PT = dw->PT;
    d.PL = dw->PL;
    d.OH = dw->OH;
    d.OW = dw->OW;
    d.act = dw->act;
    d.lo = dw->lo;
    d.hi = dw->hi;
    d.tiles_h = (dw->OH + 7) / 8;
    d.tiles_w = (dw->OW + 7) / 8;
    d.x_bytes = x_bytes;
    // 64 x 32 tiles when N fits in 32 columns (MobileNet's narrow projections), else 64 x 64
    const int bn = p.N <= 32 ? 32 : 64;
    p.tiles_m = (int)(n_img * d.tiles_h * d.tiles_w);
    p.tiles_n = (p.N + bn - 1) / bn;
    typedef void (*DwKernel)(const GemmDev, const DwDev);
    const bool s2 = dw->SH == 2;
    const DwKernel kern = bn == 32 ? (s2 ? &gemm_dw_kernel<32, 2, 1> : &gemm_dw_kernel<32, 1, 2>)
                                   : (s2 ? &gemm_dw_kernel<64, 2, 1> : &gemm_dw_kernel<64, 1, 2>);
    MGC_LAUNCH(x, kern, dim3((unsigned)(p.tiles_m * p.tiles_n)), dim3(256), 0, p, d);
}

extern "C" int mgc_hip_mbconv_supported(int Cin, int Cexp, int Cout, int stride) {
    return (Cin == 16 || Cin == 24 || Cin == 32) && Cexp > 0 && Cexp % 4 == 0 && Cexp <= kMbMaxCexp && Cout >= 1 &&
           Cout <= 32 && (stride == 1 || stride == 2);
}

extern "C" int mgc_hip_mbconv_stem_supported(int C, int KH, int KW, int Cexp, int Cout, int stride) {
    return C == kStemC && KH == kStemK && KW == kStemK && mgc_hip_mbconv_supported(32, Cexp, Cout, stride);
}

// mgc_hip_mbconv and mgc_hip_mbconv_stem: st is null for a block whose input is in memory.
static void mbconv_launch(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const mgc_hip_mbconv_args *mb,
                          const mgc_hip_stem_args *st) {
    if (g->M <= 0 || g->N <= 0) return;
    const char *const name = st ? "mgc_hip_mbconv_stem" : "mgc_hip_mbconv";
    const long ohw = (long)mb->OH * mb->OW;
    const long n_img = ohw > 0 ? g->M / ohw : 0;
    long x_bytes = n_img * mb->H * mb->W * (long)mb->Cin * 4;
    bool input_ok = aligned16(mb->x);
    if (st) {
        // bytes from img to the last element the image's strides reach
        const bool geo = st->C == kStemC && st->KH == kStemK && st->KW == kStemK && st->H > 0 && st->W > 0 &&
                         st->SH > 0 && st->SW > 0 && st->SH <= 2 && st->SW <= 2 && st->PT >= 0 && st->PL >= 0 && st->sn >= 0 && st->sc >= 0 &&
                         st->sh >= 0 && st->sw >= 0 && n_img > 0;
        x_bytes = geo ? ((n_img - 1) * st->sn + (long)(st->C - 1) * st->sc + (long)(st->H - 1) * st->sh +
                         (long)(st->W - 1) * st->sw + 1) * 4
                      : -1;
        input_ok = geo && st->img && ((uintptr_t)st->img & 3) == 0 && mb->Cin == 32;
    }
    const long b_bytes = ((long)(g->N - 1) * g->b.cs + g->K) * 4;
    const bool acts = (mb->act_e == MGC_ACT_RELU || mb->act_e == MGC_ACT_CLIP) &&
                      (mb->act_d == MGC_ACT_RELU || mb->act_d == MGC_ACT_CLIP);
    const bool ok = mgc_hip_mbconv_supported(mb->Cin, mb->Cexp, g->N, mb->SH) && mb->SH == mb->SW && acts &&
                    g->batch_rank == 0 && g->k1 == 0 && g->K == mb->Cexp && mb->H > 0 && mb->W > 0 && ohw > 0 &&
                    g->M % ohw == 0 && x_bytes > 0 && x_bytes < 0x7fffffffL && b_bytes < 0x7fffffffL &&
                    (!g->bias || g->bias_mode == 1) && g->b.kind == MGC_OP_STRIDED && g->b.rs == 1 &&
                    g->b.cs >= g->K && g->b.cs % 4 == 0 && aligned16(g->b.p) && input_ok &&
                    aligned16(mb->we) && aligned16(mb->be) && aligned16(mb->wd) && aligned16(mb->bd);
    if (!ok) {
        x->launch_error = (int)hipErrorInvalidValue;
        char msg[128];
        snprintf(msg, sizeof msg, "%s: shape, layout or alignment outside its limits", name);
        set_error(msg, hipErrorInvalidValue);
        return;
    }
    GemmDev p{};
    p.M = g->M;
    p.N = g->N;
    p.K = g->K;
    p.b = g->b;
    p.c = g->c;
    p.ldc = g->ldc;
    p.alpha = g->alpha;
    p.beta = g->beta;
    p.bias = g->bias;
    p.bias_mode = g->bias ? 1 : 0;
    p.res = g->res;
    p.ldr = g->ldr;
    p.act = g->act;
    p.lo = g->lo;
    p.hi = g->hi;
    p.split = 1;
    p.nbatch = 1;
    p.b_bytes = b_bytes;
    p.vec_out = p.ldc % 4 == 0 && aligned16(p.c) && (!p.res || (p.ldr % 4 == 0 && aligned16(p.res))) &&
                aligned16(p.bias);
    MbDev d;
    d.x = mb->x;
    d.we = mb->we;
    d.be = mb->be;
    d.wd = mb->wd;
    d.bd = mb->bd;
    d.H = mb->H;
    d.W = mb->W;
    d.Cexp = mb->Cexp;
    d.PT = mb->PT;
    d.PL = mb->PL;
    d.OH = mb->OH;
    d.OW = mb->OW;
    d.lo_e = mb->act_e == MGC_ACT_CLIP ? mb->lo_e : 0.0f;
    d.hi_e = mb->act_e == MGC_ACT_CLIP ? mb->hi_e : INFINITY;
    d.lo_d = mb->act_d == MGC_ACT_CLIP ? mb->lo_d : 0.0f;
    d.hi_d = mb->act_d == MGC_ACT_CLIP ? mb->hi_d : INFINITY;
    d.tiles_h = (mb->OH + 7) / 8;
    d.tiles_w = (mb->OW + 7) / 8;
    d.x_bytes = x_bytes;
    d.img = nullptr;
    d.iH = d.iW = d.iSH = d.iSW = d.iPT = d.iPL = 0;
    d.isn = d.isc = d.ish = d.isw = 0;
    if (st) {
        d.img = st->img;
        d.iH = st->H;
        d.iW = st->W;
        d.iSH = st->SH;
        d.iSW = st->SW;
        d.iPT = st->PT;
        d.iPL = st->PL;
        d.isn = (unsigned)st->sn;
        d.isc = (unsigned)st->sc;
        d.ish = (unsigned)st->sh;
        d.isw = (unsigned)st->sw;
    }
    const long tiles = n_img * d.tiles_h * d.tiles_w;
    typedef void (*MbKernel)(const GemmDev, const MbDev);
    const bool s2 = mb->SH == 2;
    const MbKernel kern = st               ? (s2 ? &mbconv_kernel<2, 16, true> : &mbconv_kernel<1, 16, true>)
                          : mb->Cin == 16 ? (s2 ? &mbconv_kernel<2, 8, false> : &mbconv_kernel<1, 8, false>)
                          : mb->Cin == 24 ? (s2 ? &mbconv_kernel<2, 12, false> : &mbconv_kernel<1, 12, false>)
                                          : (s2 ? &mbconv_kernel<2, 16, false> : &mbconv_kernel<1, 16, false>);
    MGC_LAUNCH(x, kern, dim3((unsigned)tiles), dim3(256), 0, p, d);
}

extern "C" void mgc_hip_mbconv(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const mgc_hip_mbconv_args *mb) {
    mbconv_launch(x, g, mb, nullptr);
}

extern "C" void mgc_hip_mbconv_stem(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const mgc_hip_mbconv_args *mb,
                                    const mgc_hip_stem_args *st) {
    if (!st) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_mbconv_stem: no stem arguments", hipErrorInvalidValue);
        return;
    }
    mbconv_launch(x, g, mb, st);
}

// Row blocks of 16 image pixels a wave may own and window pixels LDS holds, per input width:
// 64 and 96 channels up to 256 window pixels (a 14 x 14 image at stride 1 or 2), 160 channels
// up to 128 (a 7 x 7 image).
static bool expand_dw_fits(int Cin, int P, int window) {
    const int rbw = ((P + 15) / 16 + 3) / 4;
    if (Cin == 64 || Cin == 96) return rbw <= 4 && window <= 256;
    if (Cin == 160) return rbw <= 1 && window <= 128;
    return false;
}

extern "C" int mgc_hip_expand_dw_supported(int H, int W, int Cin, int Cexp, int stride, int OH, int OW) {
    if (H <= 0 || W <= 0 || OH <= 0 || OW <= 0 || Cexp <= 0 || Cexp % 32 || (stride != 1 && stride != 2)) return 0;
    const long window = ((long)(OH - 1) * stride + 3) * ((long)(OW - 1) * stride + 3);
    return (long)H * W <= 256 && window <= 256 && expand_dw_fits(Cin, H * W, (int)window);
}

extern "C" void mgc_hip_expand_dw(mgc_hip_exec *x, const mgc_hip_expand_dw_args *a) {
    if (a->N <= 0) return;
    const long x_bytes = (long)a->N * a->H * a->W * (long)a->Cin * 4;
    const bool acts = (a->act_e == MGC_ACT_RELU || a->act_e == MGC_ACT_CLIP) &&
                      (a->act_d == MGC_ACT_RELU || a->act_d == MGC_ACT_CLIP);
    const bool ok = mgc_hip_expand_dw_supported(a->H, a->W, a->Cin, a->Cexp, a->SH, a->OH, a->OW) && a->SH == a->SW &&
                    acts && a->PT >= 0 && a->PT <= 2 && a->PL >= 0 && a->PL <= 2 && x_bytes < 0x7fffffffL &&
                    (long)a->N * (a->Cexp / 32) < 0x7fffffffL && aligned16(a->x) && aligned16(a->we) &&
                    aligned16(a->be) && aligned16(a->wd) && aligned16(a->bd) && aligned16(a->out) && a->x && a->we &&
                    a->wd && a->out;
    if (!ok) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_expand_dw: shape, layout or alignment outside its limits", hipErrorInvalidValue);
        return;
    }
    XdDev d;
    d.x = a->x;
    d.we = a->we;
    d.be = a->be;
    d.wd = a->wd;
    d.bd = a->bd;
    d.out = a->out;
    d.H = a->H;
    d.W = a->W;
    d.Cexp = a->Cexp;
    d.PT = a->PT;
    d.PL = a->PL;
    d.OH = a->OH;
    d.OW = a->OW;
    d.HP = (a->OH - 1) * a->SH + 3;
    d.WP = (a->OW - 1) * a->SW + 3;
    d.slices = a->Cexp / 32;
    d.lo_e = a->act_e == MGC_ACT_CLIP ? a->lo_e : 0.0f;
    d.hi_e = a->act_e == MGC_ACT_CLIP ? a->hi_e : INFINITY;
    d.lo_d = a->act_d == MGC_ACT_CLIP ? a->lo_d : 0.0f;
    d.hi_d = a->act_d == MGC_ACT_CLIP ? a->hi_d : INFINITY;
    d.x_bytes = x_bytes;
    typedef void (*XdKernel)(const XdDev);
    const bool s2 = a->SH == 2;
    const XdKernel kern = a->Cin == 64   ? (s2 ? &gemm_expand_dw_kernel<2, 64, 4, 256> : &gemm_expand_dw_kernel<1, 64, 4, 256>)
                          : a->Cin == 96 ? (s2 ? &gemm_expand_dw_kernel<2, 96, 4, 256> : &gemm_expand_dw_kernel<1, 96, 4, 256>)
                                         : (s2 ? &gemm_expand_dw_kernel<2, 160, 1, 128> : &gemm_expand_dw_kernel<1, 160, 1, 128>);
    MGC_LAUNCH(x, kern, dim3((unsigned)((long)a->N * d.slices)), dim3(256), 0, d);
}

static void gemm_launch(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const LnTail *ln) {
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
    p.a2 = g->a2;
    p.k1 = g->k1;
    p.a2_bytes = 0;
    if (g->k1 > 0) {
        const mgc_hip_operand &s2 = g->a2;
        const bool ok = g->batch_rank == 0 && p.a.kind == MGC_OP_STRIDED && p.a.cs == 1 && p.a.rs % 4 == 0 &&
                        aligned16(p.a.p) && s2.kind == MGC_OP_CONV_NHWC && s2.KH == 1 && s2.KW == 1 &&
                        s2.PT == 0 && s2.PL == 0 && s2.C % 4 == 0 && s2.cg == s2.C && aligned16(s2.p) &&
                        s2.OH > 0 && s2.OW > 0 && g->k1 % 32 == 0 && g->k1 < p.K && s2.C == p.K - g->k1;
        if (!ok) {
            x->launch_error = (int)hipErrorInvalidValue;
            set_error("mgc_hip_gemm: concatenated-K operands outside their limits", hipErrorInvalidValue);
            return;
        }
        am = AM_CAT;
    } else if (p.a.kind == MGC_OP_STRIDED && p.a.cs == 1 && p.a.rs % 4 == 0 && p.K % 4 == 0 &&
               aligned16(p.a.p) && bs_div4(p.a_bs, p.batch_rank)) {
        am = AM_VEC;
    } else if (p.a.kind == MGC_OP_CONV_NHWC && p.a.cg % 4 == 0 && p.a.C % 4 == 0 &&
               aligned16(p.a.p) && bs_div4(p.a_bs, p.batch_rank)) {
        am = AM_CONV_VEC;
    }
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
    const mgc_hip_operand &img = am == AM_CAT ? p.a2 : p.a;  // the operand whose rows are pixels
    p.div_ow = make_fastdiv((unsigned)(img.OW > 0 ? img.OW : 1));
    p.div_ohw = make_fastdiv((unsigned)(img.OH * img.OW > 0 ? img.OH * img.OW : 1));
    p.div_cg = make_fastdiv((unsigned)(p.a.cg > 0 ? p.a.cg : 1));
    p.div_kw = make_fastdiv((unsigned)(p.a.KW > 0 ? p.a.KW : 1));

    // Reachable extents of the operands from their base pointers: the DMA kernels address them
    // through buffer resources with 32-bit offsets.
    long a_ext, b_ext;
    if (p.a.kind == MGC_OP_CONV_NHWC) {
        const long ohw = (long)p.a.OH * p.a.OW;
        const long n_img = ohw > 0 ? (p.M + ohw - 1) / ohw : 0;
        a_ext = n_img * p.a.H * p.a.W * p.a.C - (p.a.C - p.a.cg);
    } else if (am == AM_CAT) {
        a_ext = (long)(p.M - 1) * p.a.rs + (long)(p.k1 - 1) * p.a.cs + 1;
        const long ohw = (long)p.a2.OH * p.a2.OW;
        p.a2_bytes = (p.M + ohw - 1) / ohw * p.a2.H * p.a2.W * p.a2.C * 4;
    } else {
        a_ext = (long)(p.M - 1) * p.a.rs + (long)(p.K - 1) * p.a.cs + 1;
    }
    b_ext = (long)(p.K - 1) * p.b.rs + (long)(p.N - 1) * p.b.cs + 1;
    for (int d = 0; d < p.batch_rank; ++d) {
        a_ext += (long)(p.bdims[d] - 1) * p.a_bs[d];
        b_ext += (long)(p.bdims[d] - 1) * p.b_bs[d];
    }
    p.a_bytes = a_ext * 4;
    p.b_bytes = b_ext * 4;
    p.nbatch = batch;
    const long kMaxRes = 0x7fffffffL;  // buffer offsets past this mean "masked"
    bool nonneg = p.a.rs >= 0 && p.a.cs >= 0 && p.b.rs >= 0 && p.b.cs >= 0 && p.ldc >= 0 &&
                  p.ldr >= 0;
    for (int d = 0; d < p.batch_rank; ++d)
        nonneg = nonneg && p.a_bs[d] >= 0 && p.b_bs[d] >= 0 && p.c_bs[d] >= 0 && p.r_bs[d] >= 0;
    const bool dma_ok = nonneg && (am == AM_VEC || am == AM_CONV_VEC || am == AM_CAT) && bm == BD_NK_VEC &&
                        p.K > 0 && p.a_bytes > 0 && p.a_bytes < kMaxRes && p.b_bytes > 0 &&
                        p.b_bytes < kMaxRes && (am != AM_CAT || (p.a2_bytes > 0 && p.a2_bytes < kMaxRes));
    const bool stream_conv = am == AM_CONV_VEC && p.a.cg == p.a.C && p.K == p.a.KH * p.a.KW * p.a.C && p.K <= 48;
    const bool stream_ok = dma_ok && (am == AM_VEC ? p.K <= 32 : stream_conv) && !ln && batch == 1 &&
                           p.bias_mode != 2 && stream_act(p.act) && p.ldc >= p.N && (long)p.M * p.ldc * 4 < kMaxRes &&
                           (!p.res || (long)p.M * p.ldr * 4 < kMaxRes);
    if (am == AM_CAT && !dma_ok) {  // only the DMA kernels read a second source
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_gemm: concatenated-K GEMM needs a packed [N][K] B and extents below 2 GiB",
                  hipErrorInvalidValue);
        return;
    }

    // The kernel family and K split: the library's choice from the shape, or the caller's
    // (g->kernel, g->split_k), checked against what that family accepts.
    int fam;
    if (g->kernel == MGC_GEMM_AUTO || ln) {
        if (stream_ok && g->split_k <= 0 &&
            (am == AM_VEC ? use_stream(p.M, p.N, p.K) : use_stream_conv(p.M, p.N, p.K))) {
            fam = MGC_GEMM_STREAM;
        } else {
            int wsk = dma_ok && !ln && g->split_k <= 0 ? wave_split(p.M, p.N, p.K, batch) : 0;
            if (wsk > 1 && (g->workspace == nullptr || g->workspace_floats < (long)wsk * p.M * p.N)) wsk = 1;
            if (dma_ok && ln && batch == 1 && p.split >= 2) wsk = wave_split_ln(p.M, p.N, p.K, p.split);
            const int s16 = wsk > 0 && !ln && batch == 1 ? use_tile16(p.M, p.N, p.K, wsk) : 0;
            if (s16 > 0) wsk = s16;
            if (wsk > 0) p.split = wsk;
            fam = s16 > 0 ? MGC_GEMM_WSPLIT16
                  : wsk > 0 ? MGC_GEMM_WSPLIT
                  : dma_ok && narrow_tiles(p.N, p.split) ? MGC_GEMM_NARROW
                  : dma_ok ? MGC_GEMM_TILED
                           : MGC_GEMM_REGISTER;
            if (fam == MGC_GEMM_TILED && p.split == 1 && batch == 1 && quarter_tiles_ok(am, p)) {
                const int tiles = ((p.M + 63) / 64) * ((p.N + 63) / 64);
                const int rest = tiles % kCUs;
                if (tiles >= kCUs && rest > 0 && p.K >= kQuarterMinK &&
                    (rest <= kQuarterTiles || (rest <= kQuarterTilesDeepK && p.K >= kHalfQuarterMinK))) {
                    fam = MGC_GEMM_QUARTER;
                    p.nfull = tiles - rest;
                } else if (tiles > kCUs && tiles < 2 * kCUs && p.K >= kHalfQuarterMinK) {
                    // between one and two tiles per CU: half the tiles whole, half as quarters
                    fam = MGC_GEMM_QUARTER;
                    p.nfull = tiles / 2;
                }
            }
        }
    } else {
        fam = g->kernel;
        const int split = g->split_k > 1 ? g->split_k : 1;
        const char *why = nullptr;
        if (fam < MGC_GEMM_TILED || fam > MGC_GEMM_REGISTER)
            why = "unknown kernel family";
        else if (split > 1 && (batch != 1 || g->workspace == nullptr || g->workspace_floats < (long)split * p.M * p.N))
            why = "a K split needs batch 1 and split_k * M * N floats of workspace";
        else if (fam != MGC_GEMM_REGISTER && fam != MGC_GEMM_STREAM && !dma_ok)
            why = "the DMA kernels need k-contiguous operands (row-major A or NHWC image with 16-byte rows, "
                  "packed [N][K] B, K % 4 == 0) below 2 GiB";
        else if (fam == MGC_GEMM_QUARTER && (split > 1 || batch != 1 || !quarter_tiles_ok(am, p)))
            why = "quarter tiles need batch 1, no K split and 64-channel convolution groups";
        else if (fam == MGC_GEMM_STREAM && !(stream_ok && split == 1))
            why = "the streaming kernel needs a row-major A with K <= 32 or an NHWC image of one channel group "
                  "with K <= 48, batch 1, no K split, a column bias and activation none, relu or clip";
        else if (fam == MGC_GEMM_REGISTER && am == AM_CAT)
            why = "a concatenated-K GEMM runs on the DMA kernels only";
        if (why) {
            char msg[300];
            snprintf(msg, sizeof msg, "mgc_hip_gemm: kernel family %d: %s", fam, why);
            x->launch_error = (int)hipErrorInvalidValue;
            set_error(msg, hipErrorInvalidValue);
            return;
        }
        p.split = split;
        if (fam == MGC_GEMM_QUARTER) {
            // the second half of the tiles (at least one) as quarters
            const int tiles = ((p.M + 63) / 64) * ((p.N + 63) / 64);
            p.nfull = tiles / 2;
        }
    }
    if (fam == MGC_GEMM_STREAM) {
        stream_launch(x, p);
        return;
    }
    p.kchunk = ((p.K + p.split - 1) / p.split + 31) / 32 * 32;
    if (p.kchunk == 0) p.kchunk = 32;
    const int bm_t = fam == MGC_GEMM_WSPLIT16 ? 16 : fam == MGC_GEMM_WSPLIT ? 32 : fam == MGC_GEMM_NARROW ? 128 : 64;
    const int bn_t = fam == MGC_GEMM_WSPLIT16 ? 16 : fam == MGC_GEMM_WSPLIT || fam == MGC_GEMM_NARROW ? 32 : 64;
    p.tiles_m = (p.M + bm_t - 1) / bm_t;
    p.tiles_n = (p.N + bn_t - 1) / bn_t;
    GemmKernel kern = fam == MGC_GEMM_WSPLIT16 ? pick_wsplit16(am, p.kchunk)
                      : fam == MGC_GEMM_WSPLIT ? pick_wsplit(am)
                      : fam == MGC_GEMM_NARROW ? pick_dma<128, 32, 4>(am)
                      : fam == MGC_GEMM_QUARTER ? pick_dma_tail(am)
                      : fam == MGC_GEMM_TILED ? pick_dma<64, 64, 2>(am)
                                              : pick_kernel<64, 64, 2>(am, bm);
    const int threads = fam == MGC_GEMM_WSPLIT16 ? 64 * wsplit16_waves(p.kchunk) : 256;
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)(batch * p.split));
    if (fam == MGC_GEMM_QUARTER) grid.x = (unsigned)(p.nfull + 4 * (p.tiles_m * p.tiles_n - p.nfull));
    if (ln && p.split < 2) {  // the workspace did not allow the split the reduction needs
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_gemm_layer_norm: no K split", hipErrorInvalidValue);
        return;
    }
    MGC_LAUNCH(x, kern, grid, dim3(threads), 0, p);
    if (ln) {
        // a wavefront per row; one-wave workgroups when there are few rows, to spread them over CUs
        const int rows_per_block = p.M >= 1024 ? 4 : 1;
        MGC_LAUNCH(x, gemm_splitk_layer_norm, dim3((unsigned)((p.M + rows_per_block - 1) / rows_per_block)),
                   dim3(64 * rows_per_block), 0, p, (const float4 *)ln->scale, (const float4 *)ln->bias, ln->eps,
                   (float4 *)ln->out);
    } else if (p.split > 1) {
        const long total = (long)p.M * p.N;
        if (p.vec_out && p.N % 4 == 0 && total < 0x7fffffffL && aligned16(p.ws)) {
            MGC_LAUNCH(x, gemm_splitk_reduce_vec4, dim3(blocks_for(total / 4, 256, 4096)), dim3(256), 0,
                       p, make_fastdiv((unsigned)(p.N / 4)));
        } else {
            MGC_LAUNCH(x, gemm_splitk_reduce, dim3(blocks_for(total, 256, 4096)), dim3(256), 0, p);
        }
    }
}
