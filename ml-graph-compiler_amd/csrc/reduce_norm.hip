// Reductions, softmax, layer normalization, pooling and depthwise convolution.
//
// All of these are HBM-bound on MI355X. Rows are mapped to whole wavefronts (64 lanes) when the
// reduced axis is contiguous, with shuffle reductions; when the reduced axis is strided, one
// thread owns one output and walks the axis while neighbouring threads read neighbouring
// addresses, so every access is coalesced. Semantics follow the reference's C runtime
// (src/ml_graph_compiler/codegen/runtime/mgc_kernels.c:405-679): float accumulation for
// mean/max pooling and softmax, two-pass float LayerNorm, double accumulation for the generic
// float sum/mean/prod reduction (codegen/c.py:736-799).
#include "mgc_device.h"

namespace mgc {

// ---- mean / max over the middle axis ---------------------------------------------------------
__global__ void reduce_mid_strided(int is_max, long outer, long n, long inner, const float *in,
                                   float *out) {
    const long total = outer * inner;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        const long o = idx / inner, i = idx - (idx / inner) * inner;
        const float *src = in + o * n * inner + i;
        float acc = is_max ? -INFINITY : 0.0f;
        for (long k = 0; k < n; ++k) {
            float v = src[k * inner];
            acc = is_max ? (v > acc ? v : acc) : acc + v;
        }
        if (!is_max) acc *= n > 0 ? 1.0f / (float)n : 0.0f;
        out[idx] = acc;
    }
}

// inner % 4 == 0 (global pooling over NHWC): workgroup (x, o) owns CQ column quads of row
// block o, and its 256 / CQ row parts each walk every (256 / CQ)-th of the n rows with 16-byte
// loads, four rows' loads in flight at a time, then the parts' results meet in LDS in part
// order. CQ = 16 (16 parts) for long rows such as a 7 x 7 pooling window, so each thread reads
// about n / 16 rows in one or two memory round trips and even batch 1 runs many workgroups.
template <int CQ>
__global__ void __launch_bounds__(256) reduce_mid_vec4(int is_max, int n, int inner4, const float4 *in,
                                                       float4 *out) {
    constexpr int P = 256 / CQ;
    const int cq = threadIdx.x % CQ, part = threadIdx.x / CQ;
    const int col = blockIdx.x * CQ + cq;
    const long o = blockIdx.y;
    const float init = is_max ? -INFINITY : 0.0f;
    float4 acc = make_float4(init, init, init, init);
    auto fold = [&](const float4 v) __attribute__((always_inline)) {
        if (is_max) {
            acc.x = v.x > acc.x ? v.x : acc.x;
            acc.y = v.y > acc.y ? v.y : acc.y;
            acc.z = v.z > acc.z ? v.z : acc.z;
            acc.w = v.w > acc.w ? v.w : acc.w;
        } else {
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
    };
    if (col < inner4) {
        const float4 *src = in + o * n * inner4 + col;
        for (int k0 = part; k0 < n; k0 += 4 * P) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                v[u] = k0 + u * P < n ? src[(long)(k0 + u * P) * inner4] : make_float4(init, init, init, init);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (k0 + u * P < n) fold(v[u]);
        }
    }
    __shared__ float4 partial[P][CQ];
    partial[part][cq] = acc;
    __syncthreads();
    if (part != 0 || col >= inner4) return;
    for (int q = 1; q < P; ++q) fold(partial[q][cq]);
    if (!is_max) {
        const float s = n > 0 ? 1.0f / (float)n : 0.0f;
        acc.x *= s;
        acc.y *= s;
        acc.z *= s;
        acc.w *= s;
    }
    out[o * inner4 + col] = acc;
}

// inner == 1: one wavefront per row.
__global__ void reduce_mid_rows(int is_max, long outer, long n, const float *in, float *out) {
    const int lane = threadIdx.x & 63;
    const long wave = (blockIdx.x * (long)blockDim.x + threadIdx.x) >> 6;
    const long waves = ((long)gridDim.x * blockDim.x) >> 6;
    for (long o = wave; o < outer; o += waves) {
        const float *src = in + o * n;
        float acc = is_max ? -INFINITY : 0.0f;
        for (long k = lane; k < n; k += 64) {
            float v = src[k];
            acc = is_max ? fmaxf(acc, v) : acc + v;
        }
        acc = is_max ? wave_max(acc) : wave_sum(acc);
        if (lane == 0) out[o] = is_max ? acc : acc * (n > 0 ? 1.0f / (float)n : 0.0f);
    }
}

// ---- generic reduction (sum, mean, max, min, prod) -----------------------------------------
template <typename T, typename Acc>
__global__ void reduce_generic(int kind, long outer, long n, long inner, const T *in, T *out) {
    const long total = outer * inner;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        const long o = idx / inner, i = idx - (idx / inner) * inner;
        const T *src = in + o * n * inner + i;
        Acc acc;
        if (kind == 2)
            acc = (Acc)src[0];
        else if (kind == 3)
            acc = (Acc)src[0];
        else if (kind == 4)
            acc = (Acc)1;
        else
            acc = (Acc)0;
        for (long k = 0; k < n; ++k) {
            Acc v = (Acc)src[k * inner];
            if (kind == 0 || kind == 1)
                acc += v;
            else if (kind == 2)
                acc = v > acc ? v : acc;
            else if (kind == 3)
                acc = v < acc ? v : acc;
            else
                acc *= v;
        }
        if (kind == 1) acc = acc / (Acc)n;
        out[idx] = (T)acc;
    }
}

template <typename T>
__global__ void argmax_kernel(long outer, long n, long inner, const T *in, long long *out) {
    const long total = outer * inner;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        const long o = idx / inner, i = idx - (idx / inner) * inner;
        const T *src = in + o * n * inner + i;
        long best = 0;
        T bv = src[0];
        for (long k = 1; k < n; ++k) {
            T v = src[k * inner];
            if (v > bv) {
                bv = v;
                best = k;
            }
        }
        out[idx] = best;
    }
}

// ---- softmax ----------------------------------------------------------------------------------
// inner == 1: one wavefront per row, the row cached in registers when it fits (n <= 64 * 16).
__global__ void __launch_bounds__(256) softmax_rows(long outer, long n, const float *in,
                                                    float *out, int log_softmax) {
    constexpr int CACHE = 16;
    const int lane = threadIdx.x & 63;
    const long wave = (blockIdx.x * (long)blockDim.x + threadIdx.x) >> 6;
    const long waves = ((long)gridDim.x * blockDim.x) >> 6;
    const bool cached = n <= 64 * CACHE;
    for (long o = wave; o < outer; o += waves) {
        const float *src = in + o * n;
        float *dst = out + o * n;
        float v[CACHE];
        float m = -INFINITY;
        if (cached) {
#pragma unroll
            for (int j = 0; j < CACHE; ++j) {
                long k = lane + 64L * j;
                v[j] = k < n ? src[k] : -INFINITY;
                m = fmaxf(m, v[j]);
            }
        } else {
            for (long k = lane; k < n; k += 64) m = fmaxf(m, src[k]);
        }
        m = wave_max(m);
        float s = 0.0f;
        if (cached) {
#pragma unroll
            for (int j = 0; j < CACHE; ++j) {
                long k = lane + 64L * j;
                float e = k < n ? expf(v[j] - m) : 0.0f;
                s += e;
                v[j] = e;
            }
        } else {
            for (long k = lane; k < n; k += 64) s += expf(src[k] - m);
        }
        s = wave_sum(s);
        if (log_softmax) {
            const float ls = logf(s);
            for (long k = lane; k < n; k += 64) dst[k] = src[k] - m - ls;
        } else {
            const float inv = 1.0f / s;
            if (cached) {
#pragma unroll
                for (int j = 0; j < CACHE; ++j) {
                    long k = lane + 64L * j;
                    if (k < n) dst[k] = v[j] * inv;
                }
            } else {
                for (long k = lane; k < n; k += 64) dst[k] = expf(src[k] - m) * inv;
            }
        }
    }
}

// inner > 1: one thread per (outer, inner) position walks the strided axis.
__global__ void softmax_strided(long outer, long n, long inner, const float *in, float *out,
                                int log_softmax) {
    const long total = outer * inner;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        const long o = idx / inner, i = idx - (idx / inner) * inner;
        const float *src = in + o * n * inner + i;
        float *dst = out + o * n * inner + i;
        float m = -INFINITY;
        for (long k = 0; k < n; ++k) m = fmaxf(m, src[k * inner]);
        float s = 0.0f;
        for (long k = 0; k < n; ++k) s += expf(src[k * inner] - m);
        if (log_softmax) {
            const float ls = logf(s);
            for (long k = 0; k < n; ++k) dst[k * inner] = src[k * inner] - m - ls;
        } else {
            const float inv = 1.0f / s;
            for (long k = 0; k < n; ++k) dst[k * inner] = expf(src[k * inner] - m) * inv;
        }
    }
}

// ---- layer normalization: one wavefront per row ------------------------------------------------
__global__ void __launch_bounds__(256) layer_norm_rows(long rows, long cols, const float *in,
                                                       const float *scale, const float *bias,
                                                       float eps, float *out) {
    constexpr int CACHE = 16;
    const int lane = threadIdx.x & 63;
    const long wave = (blockIdx.x * (long)blockDim.x + threadIdx.x) >> 6;
    const long waves = ((long)gridDim.x * blockDim.x) >> 6;
    const bool cached = cols <= 64 * CACHE;
    for (long r = wave; r < rows; r += waves) {
        const float *src = in + r * cols;
        float *dst = out + r * cols;
        float v[CACHE];
        float sum = 0.0f;
        if (cached) {
#pragma unroll
            for (int j = 0; j < CACHE; ++j) {
                long k = lane + 64L * j;
                v[j] = k < cols ? src[k] : 0.0f;
                sum += v[j];
            }
        } else {
            for (long k = lane; k < cols; k += 64) sum += src[k];
        }
        const float mean = wave_sum(sum) / (float)cols;
        float var = 0.0f;
        if (cached) {
#pragma unroll
            for (int j = 0; j < CACHE; ++j) {
                long k = lane + 64L * j;
                float d = k < cols ? v[j] - mean : 0.0f;
                var += d * d;
            }
        } else {
            for (long k = lane; k < cols; k += 64) {
                float d = src[k] - mean;
                var += d * d;
            }
        }
        const float inv = 1.0f / sqrtf(wave_sum(var) / (float)cols + eps);
        if (cached) {
#pragma unroll
            for (int j = 0; j < CACHE; ++j) {
                long k = lane + 64L * j;
                if (k < cols) {
                    float y = (v[j] - mean) * inv;
                    if (scale) y *= scale[k];
                    if (bias) y += bias[k];
                    dst[k] = y;
                }
            }
        } else {
            for (long k = lane; k < cols; k += 64) {
                float y = (src[k] - mean) * inv;
                if (scale) y *= scale[k];
                if (bias) y += bias[k];
                dst[k] = y;
            }
        }
    }
}

// cols % 4 == 0 and cols <= 1024 with 16-byte aligned rows (the hidden sizes of transformer
// encoders): one wavefront per row holds the row in registers as up to four float4 per lane, so
// the row is read once and written once with 16-byte accesses and three times fewer load
// instructions than the scalar kernel.
__global__ void __launch_bounds__(256) layer_norm_rows_vec4(int rows, int cols4, const float4 *in,
                                                            const float4 *scale, const float4 *bias,
                                                            float eps, float4 *out) {
    const int lane = threadIdx.x & 63;
    const int r = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (r >= rows) return;
    const float4 *src = in + (long)r * cols4;
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = lane + 64 * j;
        v[j] = k < cols4 ? src[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const LnAffine aff = ln_affine_load(lane, cols4, scale, bias);
    layer_norm_row_vec4(v, lane, cols4, aff, eps, out + (long)r * cols4);
}

// Embedding lookup, the addend and the LayerNorm in one pass (a transformer encoder's input:
// Gather of the token table, codegen/c.py:662-688, the Add of the position / segment embeddings,
// c.py:360-529, and mgc_layer_norm, mgc_runtime.h:199-200): one wavefront per output row r takes
// row ids[r] of the table and row r % add_rows of the addend (a full-shape addend or one that
// repeats over the leading dimensions), adds them and normalizes the sum from registers with
// layer_norm_row_vec4, so it rounds as the Add and the LayerNorm kernel do apart; when the sum
// is read elsewhere too (GPT-2's first residual) it is also stored (sum_out). An index out of
// range sets the flag and leaves its row unwritten, as gather_rows16_kernel does.
__global__ void __launch_bounds__(256) gather_add_layer_norm_rows(long rows, int cols4, const float4 *table, long dim,
                                                                  const void *idx, int idx_dtype,
                                                                  const float4 *addend, long add_rows,
                                                                  const float4 *scale, const float4 *bias,
                                                                  float eps, float4 *out, float4 *sum_out,
                                                                  int *flag) {
    const int lane = threadIdx.x & 63;
    const long r = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (r >= rows) return;
    long k = idx_dtype == MGC_I64 ? static_cast<const long long *>(idx)[r] : (long)static_cast<const int *>(idx)[r];
    if (k < 0) k += dim;
    if (k < 0 || k >= dim) {
        if (lane == 0) *flag = 1;
        return;
    }
    const float4 *src = table + k * cols4;
    const float4 *add = addend ? addend + (r % add_rows) * cols4 : nullptr;
    const LnAffine aff = ln_affine_load(lane, cols4, scale, bias);
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int q = lane + 64 * j;
        v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (q < cols4) {
            v[j] = src[q];
            if (add) {
                const float4 a = add[q];
                v[j].x += a.x;
                v[j].y += a.y;
                v[j].z += a.z;
                v[j].w += a.w;
            }
        }
    }
    if (sum_out) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j < cols4) sum_out[r * cols4 + lane + 64 * j] = v[j];
    }
    layer_norm_row_vec4(v, lane, cols4, aff, eps, out + r * cols4);
}

// ---- pooling -----------------------------------------------------------------------------------
struct PoolGeo {
    int N, H, W, C, KH, KW, SH, SW, DH, DW, PT, PL, PB, PR, OH, OW, include_pad, is_max;
};

__device__ __forceinline__ int window_count(const PoolGeo &g, int oh, int ow) {
    int count = 0;
    for (int kh = 0; kh < g.KH; ++kh) {
        int ih = oh * g.SH - g.PT + kh * g.DH;
        bool in_h = g.include_pad ? (ih >= -g.PT && ih < g.H + g.PB) : (ih >= 0 && ih < g.H);
        if (!in_h) continue;
        for (int kw = 0; kw < g.KW; ++kw) {
            int iw = ow * g.SW - g.PL + kw * g.DW;
            bool in_w = g.include_pad ? (iw >= -g.PL && iw < g.W + g.PR) : (iw >= 0 && iw < g.W);
            if (in_w) ++count;
        }
    }
    return count;
}

__global__ void pool_nhwc(const PoolGeo g, const float *in, float *out) {
    const long total = (long)g.N * g.OH * g.OW * g.C;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        long t = idx;
        const int c = (int)(t % g.C);
        t /= g.C;
        const int ow = (int)(t % g.OW);
        t /= g.OW;
        const int oh = (int)(t % g.OH);
        const int n = (int)(t / g.OH);
        const float *img = in + (long)n * g.H * g.W * g.C + c;
        float acc = g.is_max ? -INFINITY : 0.0f;
        for (int kh = 0; kh < g.KH; ++kh) {
            int ih = oh * g.SH - g.PT + kh * g.DH;
            if (ih < 0 || ih >= g.H) continue;
            for (int kw = 0; kw < g.KW; ++kw) {
                int iw = ow * g.SW - g.PL + kw * g.DW;
                if (iw < 0 || iw >= g.W) continue;
                float v = img[((long)ih * g.W + iw) * g.C];
                acc = g.is_max ? (v > acc ? v : acc) : acc + v;
            }
        }
        if (!g.is_max) {
            int cnt = window_count(g, oh, ow);
            acc *= cnt > 0 ? 1.0f / (float)cnt : 0.0f;
        }
        out[idx] = acc;
    }
}

// NHWC with C % 4 == 0: one thread per output channel quad, 16-byte loads and stores, 32-bit
// index arithmetic with host-computed divisors (the element count is below 2^31).
// K > 0: a K x K window whose K * K loads are all requested (addresses clamped into the image)
// before the first is combined; K == 0: any window.
template <int K>
__global__ void pool_nhwc_vec4(const PoolGeo g, FastDiv div_c4, FastDiv div_ow, FastDiv div_oh,
                               int total, const float *in, float *out) {
    const int C4 = g.C >> 2;
    const int KH = K > 0 ? K : g.KH, KW = K > 0 ? K : g.KW;
    for (int idx = xcd_block() * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        int t = fdiv(idx, div_c4);
        const int c4 = idx - t * C4;
        int t2 = fdiv(t, div_ow);
        const int ow = t - t2 * g.OW;
        const int n = fdiv(t2, div_oh);
        const int oh = t2 - n * g.OH;
        const float *img = in + (long)n * g.H * g.W * g.C + c4 * 4;
        const float init = g.is_max ? -INFINITY : 0.0f;
        float4 acc = make_float4(init, init, init, init);
        if (K > 0) {
            // every tap's load first (addresses clamped into the image), then the combine: taps
            // outside the image are skipped, as below
            float4 v[K > 0 ? K : 1][K > 0 ? K : 1];
            bool ok[K > 0 ? K : 1][K > 0 ? K : 1];
#pragma unroll
            for (int kh = 0; kh < K; ++kh) {
                const int ih = oh * g.SH - g.PT + kh * g.DH;
                const int ihc = min(max(ih, 0), g.H - 1);
#pragma unroll
                for (int kw = 0; kw < K; ++kw) {
                    const int iw = ow * g.SW - g.PL + kw * g.DW;
                    ok[kh][kw] = (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W;
                    v[kh][kw] = *reinterpret_cast<const float4 *>(img + (long)(ihc * g.W + min(max(iw, 0), g.W - 1)) * g.C);
                }
            }
#pragma unroll
            for (int kh = 0; kh < K; ++kh)
#pragma unroll
                for (int kw = 0; kw < K; ++kw) {
                    if (!ok[kh][kw]) continue;
                    const float4 x = v[kh][kw];
                    if (g.is_max) {
                        acc.x = x.x > acc.x ? x.x : acc.x;
                        acc.y = x.y > acc.y ? x.y : acc.y;
                        acc.z = x.z > acc.z ? x.z : acc.z;
                        acc.w = x.w > acc.w ? x.w : acc.w;
                    } else {
                        acc.x += x.x;
                        acc.y += x.y;
                        acc.z += x.z;
                        acc.w += x.w;
                    }
                }
        }
#pragma unroll
        for (int kh = 0; kh < (K > 0 ? 0 : KH); ++kh) {
            const int ih = oh * g.SH - g.PT + kh * g.DH;
            if (ih < 0 || ih >= g.H) continue;
#pragma unroll
            for (int kw = 0; kw < KW; ++kw) {
                const int iw = ow * g.SW - g.PL + kw * g.DW;
                if (iw < 0 || iw >= g.W) continue;
                const float4 v = *reinterpret_cast<const float4 *>(img + (long)(ih * g.W + iw) * g.C);
                if (g.is_max) {
                    acc.x = v.x > acc.x ? v.x : acc.x;
                    acc.y = v.y > acc.y ? v.y : acc.y;
                    acc.z = v.z > acc.z ? v.z : acc.z;
                    acc.w = v.w > acc.w ? v.w : acc.w;
                } else {
                    acc.x += v.x;
                    acc.y += v.y;
                    acc.z += v.z;
                    acc.w += v.w;
                }
            }
        }
        if (!g.is_max) {
            const int cnt = window_count(g, oh, ow);
            const float s = cnt > 0 ? 1.0f / (float)cnt : 0.0f;
            acc.x *= s;
            acc.y *= s;
            acc.z *= s;
            acc.w *= s;
        }
        reinterpret_cast<float4 *>(out)[idx] = acc;
    }
}

__global__ void pool_nchw(const PoolGeo g, const float *in, float *out) {
    const long total = (long)g.N * g.C * g.OH * g.OW;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        long t = idx;
        const int ow = (int)(t % g.OW);
        t /= g.OW;
        const int oh = (int)(t % g.OH);
        const long plane = t / g.OH;
        const float *img = in + plane * g.H * g.W;
        float acc = g.is_max ? -INFINITY : 0.0f;
        for (int kh = 0; kh < g.KH; ++kh) {
            int ih = oh * g.SH - g.PT + kh * g.DH;
            if (ih < 0 || ih >= g.H) continue;
            for (int kw = 0; kw < g.KW; ++kw) {
                int iw = ow * g.SW - g.PL + kw * g.DW;
                if (iw < 0 || iw >= g.W) continue;
                float v = img[(long)ih * g.W + iw];
                acc = g.is_max ? (v > acc ? v : acc) : acc + v;
            }
        }
        if (!g.is_max) {
            int cnt = window_count(g, oh, ow);
            acc = cnt > 0 ? acc / (float)cnt : 0.0f;
        }
        out[idx] = acc;
    }
}

// ---- depthwise convolution ---------------------------------------------------------------------
struct DwGeo {
    int N, H, W, C, KH, KW, SH, SW, DH, DW, PT, PL, OH, OW, act;
    float lo, hi;
};

// NHWC, four channels per thread (C % 4 == 0): float4 loads of input, weights and bias, and
// 32-bit index arithmetic with host-computed divisors (the quad count is below 2^31): 64-bit
// division chains would make this bandwidth-bound kernel ALU-bound. Blocks run in XCD order.
__global__ void depthwise_nhwc_vec4(const DwGeo g, FastDiv div_c4, FastDiv div_ow, FastDiv div_oh,
                                    int total, const float *in, const float *w, const float *bias,
                                    const float *res, float *out) {
    const int C4 = g.C >> 2;
    for (int idx = xcd_block() * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const int t = fdiv(idx, div_c4);
        const int c4 = idx - t * C4;
        const int t2 = fdiv(t, div_ow);
        const int ow = t - t2 * g.OW;
        const int n = fdiv(t2, div_oh);
        const int oh = t2 - n * g.OH;
        const int c = c4 * 4;
        float4 acc = bias ? *reinterpret_cast<const float4 *>(bias + c) : make_float4(0, 0, 0, 0);
        const float *img = in + (long)n * g.H * g.W * g.C + c;
        for (int kh = 0; kh < g.KH; ++kh) {
            const int ih = oh * g.SH - g.PT + kh * g.DH;
            if (ih < 0 || ih >= g.H) continue;
            for (int kw = 0; kw < g.KW; ++kw) {
                const int iw = ow * g.SW - g.PL + kw * g.DW;
                if (iw < 0 || iw >= g.W) continue;
                const float4 xv = *reinterpret_cast<const float4 *>(img + (long)(ih * g.W + iw) * g.C);
                const float4 wv = *reinterpret_cast<const float4 *>(w + (kh * g.KW + kw) * g.C + c);
                acc.x = fmaf(xv.x, wv.x, acc.x);
                acc.y = fmaf(xv.y, wv.y, acc.y);
                acc.z = fmaf(xv.z, wv.z, acc.z);
                acc.w = fmaf(xv.w, wv.w, acc.w);
            }
        }
        const long o = (long)idx * 4;
        if (res) {
            const float4 rv = *reinterpret_cast<const float4 *>(res + o);
            acc.x += rv.x;
            acc.y += rv.y;
            acc.z += rv.z;
            acc.w += rv.w;
        }
        acc.x = apply_act(acc.x, g.act, g.lo, g.hi);
        acc.y = apply_act(acc.y, g.act, g.lo, g.hi);
        acc.z = apply_act(acc.z, g.act, g.lo, g.hi);
        acc.w = apply_act(acc.w, g.act, g.lo, g.hi);
        *reinterpret_cast<float4 *>(out + o) = acc;
    }
}

// 3x3, dilation 1, horizontal stride SW (1 or 2), C % 4 == 0: each thread computes four
// channels of T neighbouring output pixels of one row. The ((T - 1) * SW + 3) input columns
// those outputs share are loaded once per kernel row and the weights once per thread, so the
// cache traffic per output quad drops from 18 float4 loads (nine input taps and nine weights)
// to (3 * ((T - 1) * SW + 3) + 9) / T. Blocks run in XCD order (xcd_block), so the three input
// rows an output row needs are mostly fetched into one L2 once. Taps are accumulated in the
// same order as the general kernel (bias, then row-major over the window), and out-of-image
// taps are skipped, not multiplied.
template <int SW, int T>
__global__ void __launch_bounds__(256) depthwise3x3_nhwc_vec4(const DwGeo g, FastDiv div_c4, FastDiv div_owb,
                                                              FastDiv div_oh, int total, const float *in,
                                                              const float *w, const float *bias,
                                                              const float *res, float *out) {
    constexpr int NCOL = (T - 1) * SW + 3;
    const int C4 = g.C >> 2, OWB = (g.OW + T - 1) / T;
    for (int idx = xcd_block() * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const int t = fdiv(idx, div_c4);
        const int c4 = idx - t * C4;
        const int t2 = fdiv(t, div_owb);
        const int owb = t - t2 * OWB;
        const int n = fdiv(t2, div_oh);
        const int oh = t2 - n * g.OH;
        const int c = c4 * 4, ow0 = owb * T, iw0 = ow0 * SW - g.PL;
        const float4 b = bias ? *reinterpret_cast<const float4 *>(bias + c) : make_float4(0, 0, 0, 0);
        float4 acc[T];
#pragma unroll
        for (int j = 0; j < T; ++j) acc[j] = b;
        const float *img = in + (long)n * g.H * g.W * g.C + c;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
            const int ih = oh * g.SH - g.PT + kh;
            if (ih < 0 || ih >= g.H) continue;
            const float *row = img + (long)ih * g.W * g.C;
            float4 xs[NCOL];
#pragma unroll
            for (int q = 0; q < NCOL; ++q) {
                const int iw = iw0 + q;
                xs[q] = iw >= 0 && iw < g.W ? *reinterpret_cast<const float4 *>(row + (long)iw * g.C)
                                            : make_float4(0, 0, 0, 0);
            }
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) {
                const float4 wv = *reinterpret_cast<const float4 *>(w + (kh * 3 + kw) * g.C + c);
#pragma unroll
                for (int j = 0; j < T; ++j) {
                    const int iw = iw0 + j * SW + kw;
                    if (iw < 0 || iw >= g.W) continue;
                    const float4 xv = xs[j * SW + kw];
                    acc[j].x = fmaf(xv.x, wv.x, acc[j].x);
                    acc[j].y = fmaf(xv.y, wv.y, acc[j].y);
                    acc[j].z = fmaf(xv.z, wv.z, acc[j].z);
                    acc[j].w = fmaf(xv.w, wv.w, acc[j].w);
                }
            }
        }
        const long base = ((long)(n * g.OH + oh) * g.OW + ow0) * g.C + c;
#pragma unroll
        for (int j = 0; j < T; ++j) {
            if (ow0 + j >= g.OW) break;
            const long o = base + (long)j * g.C;
            float4 v = acc[j];
            if (res) {
                const float4 rv = *reinterpret_cast<const float4 *>(res + o);
                v.x += rv.x;
                v.y += rv.y;
                v.z += rv.z;
                v.w += rv.w;
            }
            v.x = apply_act(v.x, g.act, g.lo, g.hi);
            v.y = apply_act(v.y, g.act, g.lo, g.hi);
            v.z = apply_act(v.z, g.act, g.lo, g.hi);
            v.w = apply_act(v.w, g.act, g.lo, g.hi);
            *reinterpret_cast<float4 *>(out + o) = v;
        }
    }
}

// Preloading form (stride 2, and stride 1 on wide rows): every input and weight load of a
// thread is issued before the first FMA (addresses clamped into the image; out-of-image taps
// are skipped afterwards), so the thread waits for memory once. Two outputs per thread: with
// four, the preloaded rows need enough registers to halve occupancy.
template <int SW, int T>
__global__ void __launch_bounds__(256) depthwise3x3_nhwc_preload(const DwGeo g, FastDiv div_c4, FastDiv div_owb,
                                                                 FastDiv div_oh, int total, const float *in,
                                                                 const float *w, const float *bias,
                                                                 const float *res, float *out) {
    constexpr int NCOL = (T - 1) * SW + 3;
    const int C4 = g.C >> 2, OWB = (g.OW + T - 1) / T;
    for (int idx = xcd_block() * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const int t = fdiv(idx, div_c4);
        const int c4 = idx - t * C4;
        const int t2 = fdiv(t, div_owb);
        const int owb = t - t2 * OWB;
        const int n = fdiv(t2, div_oh);
        const int oh = t2 - n * g.OH;
        const int c = c4 * 4, ow0 = owb * T, iw0 = ow0 * SW - g.PL;
        // optional operands load from a valid stand-in address and select their values later
        // (a select between a load and a constant becomes a load through a stack slot)
        float4 b = *reinterpret_cast<const float4 *>((bias ? bias : w) + c);
        if (!bias) b = make_float4(0.f, 0.f, 0.f, 0.f);
        float4 wv[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) wv[k] = *reinterpret_cast<const float4 *>(w + k * g.C + c);
        const float *img = in + (long)n * g.H * g.W * g.C + c;
        float4 xs[3][NCOL];
        bool rok[3], cok[NCOL];
#pragma unroll
        for (int q = 0; q < NCOL; ++q) cok[q] = (unsigned)(iw0 + q) < (unsigned)g.W;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
            const int ih = oh * g.SH - g.PT + kh;
            rok[kh] = (unsigned)ih < (unsigned)g.H;
            const float *row = img + (long)min(max(ih, 0), g.H - 1) * g.W * g.C;
#pragma unroll
            for (int q = 0; q < NCOL; ++q)
                xs[kh][q] = *reinterpret_cast<const float4 *>(row + (long)min(max(iw0 + q, 0), g.W - 1) * g.C);
        }
        float4 acc[T];
#pragma unroll
        for (int j = 0; j < T; ++j) acc[j] = b;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) {
#pragma unroll
                for (int j = 0; j < T; ++j) {
                    const int q = j * SW + kw;
                    // taps outside the image add nothing (the reference skips them)
                    if (!(rok[kh] && cok[q])) continue;
                    const float4 xv = xs[kh][q];
                    const float4 wk = wv[kh * 3 + kw];
                    acc[j].x = fmaf(xv.x, wk.x, acc[j].x);
                    acc[j].y = fmaf(xv.y, wk.y, acc[j].y);
                    acc[j].z = fmaf(xv.z, wk.z, acc[j].z);
                    acc[j].w = fmaf(xv.w, wk.w, acc[j].w);
                }
            }
        }
        const long base = ((long)(n * g.OH + oh) * g.OW + ow0) * g.C + c;
        // the residual quads of the thread's outputs together, then the stores (no early exit,
        // so the accumulators stay in registers)
        float4 rv[T];
#pragma unroll
        for (int j = 0; j < T; ++j)
            rv[j] = *reinterpret_cast<const float4 *>(res ? res + base + (long)min(j, g.OW - 1 - ow0) * g.C : in + c);
#pragma unroll
        for (int j = 0; j < T; ++j) {
            if (ow0 + j < g.OW) {
                float4 v = acc[j];
                if (res) {
                    v.x += rv[j].x;
                    v.y += rv[j].y;
                    v.z += rv[j].z;
                    v.w += rv[j].w;
                }
                v.x = apply_act(v.x, g.act, g.lo, g.hi);
                v.y = apply_act(v.y, g.act, g.lo, g.hi);
                v.z = apply_act(v.z, g.act, g.lo, g.hi);
                v.w = apply_act(v.w, g.act, g.lo, g.hi);
                *reinterpret_cast<float4 *>(out + base + (long)j * g.C) = v;
            }
        }
    }
}

// 3x3, dilation 1, stride S, C % 4 == 0, staged through LDS: a workgroup owns an 8 x 8 block
// of output pixels over 8 channel quads. It loads the ((8 - 1) S + 3)^2 input pixels of those
// quads once (zeros outside the image: 16-byte loads, 128 contiguous bytes per pixel), then
// each thread computes two output quads from LDS. Every input quad crosses L2 -> CU once per
// tile (the halo adds (7 S + 3)^2 / (8 S)^2 - 1) instead of once per window that covers it.
// Taps accumulate after the bias in row-major order, as in the other depthwise kernels; taps
// outside the image contribute zero products.
template <int S>
__global__ void __launch_bounds__(256) depthwise3x3_nhwc_lds(const DwGeo g, int tiles_w, int tiles_h, int cgroups,
                                                             const float *in, const float *w, const float *bias,
                                                             const float *res, float *out) {
    constexpr int T = 8, CQ = 8, IT = (T - 1) * S + 3;
    __shared__ float4 tile[IT * IT * CQ];
    int b = xcd_block();
    const int cg = b % cgroups;
    b /= cgroups;
    const int tw = b % tiles_w;
    b /= tiles_w;
    const int th = b % tiles_h;
    const int n = b / tiles_h;
    const int C4 = g.C >> 2;
    const int c4base = cg * CQ;
    const int oh0 = th * T, ow0 = tw * T;
    const int ih0 = oh0 * S - g.PT, iw0 = ow0 * S - g.PL;
    const float4 *img = reinterpret_cast<const float4 *>(in) + (long)n * g.H * g.W * C4;
    for (int e = threadIdx.x; e < IT * IT * CQ; e += 256) {
        const int q = e % CQ, pix = e / CQ;
        const int r = pix / IT, col = pix - r * IT;
        const int ih = ih0 + r, iw = iw0 + col, c4 = c4base + q;
        const bool inside = ih >= 0 && ih < g.H && iw >= 0 && iw < g.W && c4 < C4;
        tile[e] = inside ? img[((long)ih * g.W + iw) * C4 + c4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    __syncthreads();
    const int q = threadIdx.x % CQ, c4 = c4base + q;
    if (c4 >= C4) return;
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 wv[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) wv[t] = w4[t * C4 + c4];
    const float4 bv = bias ? reinterpret_cast<const float4 *>(bias)[c4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int p = threadIdx.x / CQ + 32 * k;
        const int ohl = p / T, owl = p % T;
        const int oh = oh0 + ohl, ow = ow0 + owl;
        if (oh >= g.OH || ow >= g.OW) continue;
        float4 acc = bv;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) {
                const float4 xv = tile[((ohl * S + kh) * IT + owl * S + kw) * CQ + q];
                const float4 wt = wv[kh * 3 + kw];
                acc.x = fmaf(xv.x, wt.x, acc.x);
                acc.y = fmaf(xv.y, wt.y, acc.y);
                acc.z = fmaf(xv.z, wt.z, acc.z);
                acc.w = fmaf(xv.w, wt.w, acc.w);
            }
        const long o = ((long)(n * g.OH + oh) * g.OW + ow) * C4 + c4;
        if (res) {
            const float4 rv = reinterpret_cast<const float4 *>(res)[o];
            acc.x += rv.x;
            acc.y += rv.y;
            acc.z += rv.z;
            acc.w += rv.w;
        }
        acc.x = apply_act(acc.x, g.act, g.lo, g.hi);
        acc.y = apply_act(acc.y, g.act, g.lo, g.hi);
        acc.z = apply_act(acc.z, g.act, g.lo, g.hi);
        acc.w = apply_act(acc.w, g.act, g.lo, g.hi);
        reinterpret_cast<float4 *>(out)[o] = acc;
    }
}

// 3x3, stride 1, dilation 1, C % 4 == 0, for large launches: a workgroup streams down a strip
// of output columns for a slice of at most 64 channel quads over a run of output rows. Thread
// (j, q) owns channel quad q of the slice and output columns 4 j .. 4 j + 3 of the strip (so
// the strip is 4 * floor(256 / nq) columns wide): its nine weight quads stay in registers and
// each output row costs it 18 LDS reads for four outputs. The input rows the strip reads go
// through an LDS ring of four rows: while output row k of the run (input rows counted from the
// run's first) is computed from ring rows k .. k + 2, input row k + 4 is requested into
// registers and input row k + 3, requested during output row k - 1, lands in the slot that
// row k - 1 held, so every row's latency hides behind two output rows of work and each input
// byte crosses HBM -> CU about once. Taps accumulate after the bias in row-major order and rows
// or columns outside the image add zero products, as in the other depthwise kernels.
constexpr int kDwRowsCQ = 64;     // channel quads per workgroup at most
constexpr int kDwRowsQuads = 4 * 256 + 2 * kDwRowsCQ;  // quads of a ring row at most: (4 G + 2) nq
__global__ void __launch_bounds__(256) depthwise3x3_nhwc_rows(const DwGeo g, int strips, int cgroups, int cq,
                                                              int chunks, int rows_per, const float *in,
                                                              const float *w, const float *bias, const float *res,
                                                              float *out) {
    __shared__ float4 ring[4][kDwRowsQuads];
    int b = xcd_block();
    const int cgi = b % cgroups;
    b /= cgroups;
    const int chunk = b % chunks;
    b /= chunks;
    const int strip = b % strips;
    const int n = b / strips;
    const int C4 = g.C >> 2;
    const int c4base = cgi * cq;
    const int nq = min(cq, C4 - c4base);     // quads of this slice
    const int G = 256 / nq;                  // column groups
    const int TW = 4 * G;                    // strip width
    const int IWp = TW + 2;                  // input pixels per ring row
    const int ow0 = strip * TW, iw0 = ow0 - g.PL;
    const int oh_begin = chunk * rows_per, oh_end = min(g.OH, oh_begin + rows_per);
    const float4 *img = reinterpret_cast<const float4 *>(in) + (long)n * g.H * g.W * C4 + c4base;
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const int tid = threadIdx.x;
    const int row_elems = IWp * nq;          // quads of one ring row (<= 4 * 256 + 2 * nq)
    const int per = (row_elems + 255) / 256;
    constexpr int PER_MAX = (kDwRowsQuads + 255) / 256;
    const int q = tid % nq, j = tid / nq;
    const bool worker = j < G;
    const int c4 = c4base + q;

    float4 wv[9];
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
#pragma unroll
    for (int t = 0; t < 9; ++t) wv[t] = worker ? w4[t * C4 + c4] : zero4;
    const float4 bv = worker && bias ? reinterpret_cast<const float4 *>(bias)[c4] : zero4;

    auto slot_of = [](int ih) { return (ih + 8) & 3; };
    // input row ih of the strip into registers: buffer loads over the image, an element outside
    // it (or past the slice) at an offset past the resource's end, which reads as zero
    const __amdgpu_buffer_rsrc_t rimg = __builtin_amdgcn_make_buffer_rsrc(
        (void *)img, (short)0, (int)(((long)g.H * g.W * C4 - c4base) * 16), 0x00020000);
    constexpr unsigned OOB = 0x80000000u;
    auto fetch = [&](int ih, float4 (&v)[PER_MAX]) __attribute__((always_inline)) {
        const bool row_in = ih >= 0 && ih < g.H;
#pragma unroll
        for (int k = 0; k < PER_MAX; ++k) {
            const int e = tid + 256 * k;
            const int px = e / nq, qq = e - px * nq;
            const int iw = iw0 + px;
            const bool ok = k < per && e < row_elems && row_in && iw >= 0 && iw < g.W;
            const unsigned off = ok ? (unsigned)(((ih * g.W + iw) * C4 + qq) * 16) : OOB;
            v[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rimg, off, 0, 0));
        }
    };
    auto place = [&](int slot, const float4 (&v)[PER_MAX]) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < PER_MAX; ++k) {
            const int e = tid + 256 * k;
            if (k < per && e < row_elems) ring[slot][e] = v[k];
        }
    };
    // input rows oh_begin - PT .. oh_begin - PT + 3: the first output row's three and the next one
    const int ih0 = oh_begin - g.PT;
    float4 pa[PER_MAX], pb[PER_MAX];
    fetch(ih0, pa);
    fetch(ih0 + 1, pb);
    place(slot_of(ih0), pa);
    place(slot_of(ih0 + 1), pb);
    fetch(ih0 + 2, pa);
    fetch(ih0 + 3, pb);
    place(slot_of(ih0 + 2), pa);
    place(slot_of(ih0 + 3), pb);
    __syncthreads();
    // one output row: request input row oh - PT + 4 into rq, compute, then place input row
    // oh - PT + 3 (requested during the previous output row, in rl) in the slot of row
    // oh - PT - 1, which the finished output row oh - 1 read last
    auto step = [&](const int oh, float4 (&rq)[PER_MAX], float4 (&rl)[PER_MAX]) __attribute__((always_inline)) {
        if (oh + 2 < oh_end) fetch(oh - g.PT + 4, rq);
        if (worker) {
            float4 acc[4] = {bv, bv, bv, bv};
#pragma unroll
            for (int kh = 0; kh < 3; ++kh) {
                const float4 *rr = ring[slot_of(oh - g.PT + kh)] + 4 * j * nq + q;
                float4 xs[6];
#pragma unroll
                for (int c = 0; c < 6; ++c) xs[c] = rr[c * nq];
#pragma unroll
                for (int kw = 0; kw < 3; ++kw) {
                    const float4 wt = wv[kh * 3 + kw];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        acc[u].x = fmaf(xs[u + kw].x, wt.x, acc[u].x);
                        acc[u].y = fmaf(xs[u + kw].y, wt.y, acc[u].y);
                        acc[u].z = fmaf(xs[u + kw].z, wt.z, acc[u].z);
                        acc[u].w = fmaf(xs[u + kw].w, wt.w, acc[u].w);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int ow = ow0 + 4 * j + u;
                if (ow >= g.OW) break;
                const long o = ((long)(n * g.OH + oh) * g.OW + ow) * C4 + c4;
                float4 v = acc[u];
                if (res) {
                    const float4 rv = reinterpret_cast<const float4 *>(res)[o];
                    v.x += rv.x;
                    v.y += rv.y;
                    v.z += rv.z;
                    v.w += rv.w;
                }
                v.x = apply_act(v.x, g.act, g.lo, g.hi);
                v.y = apply_act(v.y, g.act, g.lo, g.hi);
                v.z = apply_act(v.z, g.act, g.lo, g.hi);
                v.w = apply_act(v.w, g.act, g.lo, g.hi);
                reinterpret_cast<float4 *>(out)[o] = v;
            }
        }
        if (oh > oh_begin && oh + 1 < oh_end) place(slot_of(oh - g.PT + 3), rl);
        __syncthreads();
    };
    // the two register buffers alternate by output row; pairs keep their roles static
    for (int oh = oh_begin; oh < oh_end; oh += 2) {
        step(oh, pa, pb);
        if (oh + 1 < oh_end) step(oh + 1, pb, pa);
    }
}

__global__ void depthwise_nhwc(const DwGeo g, const float *in, const float *w, const float *bias,
                               const float *res, float *out) {
    const long total = (long)g.N * g.OH * g.OW * g.C;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        long t = idx;
        const int c = (int)(t % g.C);
        t /= g.C;
        const int ow = (int)(t % g.OW);
        t /= g.OW;
        const int oh = (int)(t % g.OH);
        const int n = (int)(t / g.OH);
        float acc = bias ? bias[c] : 0.0f;
        const float *img = in + (long)n * g.H * g.W * g.C + c;
        for (int kh = 0; kh < g.KH; ++kh) {
            int ih = oh * g.SH - g.PT + kh * g.DH;
            if (ih < 0 || ih >= g.H) continue;
            for (int kw = 0; kw < g.KW; ++kw) {
                int iw = ow * g.SW - g.PL + kw * g.DW;
                if (iw < 0 || iw >= g.W) continue;
                acc = fmaf(img[((long)ih * g.W + iw) * g.C], w[((long)kh * g.KW + kw) * g.C + c],
                           acc);
            }
        }
        if (res) acc += res[idx];
        out[idx] = apply_act(acc, g.act, g.lo, g.hi);
    }
}

__global__ void depthwise_nchw(const DwGeo g, const float *in, const float *w, const float *bias,
                               const float *res, float *out) {
    const long total = (long)g.N * g.C * g.OH * g.OW;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        long t = idx;
        const int ow = (int)(t % g.OW);
        t /= g.OW;
        const int oh = (int)(t % g.OH);
        const long plane = t / g.OH;
        const int c = (int)(plane % g.C);
        const float *img = in + plane * g.H * g.W;
        const float *wk = w + (long)c * g.KH * g.KW;
        float acc = bias ? bias[c] : 0.0f;
        for (int kh = 0; kh < g.KH; ++kh) {
            int ih = oh * g.SH - g.PT + kh * g.DH;
            if (ih < 0 || ih >= g.H) continue;
            for (int kw = 0; kw < g.KW; ++kw) {
                int iw = ow * g.SW - g.PL + kw * g.DW;
                if (iw < 0 || iw >= g.W) continue;
                acc = fmaf(img[(long)ih * g.W + iw], wk[kh * g.KW + kw], acc);
            }
        }
        if (res) acc += res[idx];
        out[idx] = apply_act(acc, g.act, g.lo, g.hi);
    }
}

// ---- global average pooling + fully connected layer, for a few images --------------------------
// out[i][f] = act(bias[f] + sum_c W[f][c] * (1 / P) sum_p x[i][p][c]) (codegen/c.py:1255-1270 then
// :974-1003: mgc_reduce_mid's mean, mgc_kernels.c:593-612, followed by mgc_gemm). Workgroup
// (fb, i), 16 waves: wave v owns output f = 16 fb + v. Its weight row is requested first (lane l
// holds quads l + 64 j), so that latency overlaps the pooling. Pooling of image i: thread t sums
// channel quad q = t % C4 over pixels part, part + parts, ... (part = t / C4, parts = 1024 / C4),
// eight 16-byte buffer loads in flight at a time (sixteen measured no faster); the parts meet in
// LDS in part order and are scaled by 1 / P. Each wave then forms its dot product (lane l over
// its quads in order, then a fixed butterfly over the 64 lanes). One launch instead of a pooling
// launch and a GEMM launch; every workgroup reads the whole image, so it suits batch 1-4 (the
// image is 0.2-0.4 MB for ResNet-50 and MobileNetV2).
constexpr int kPfThreads = 1024, kPfOut = kPfThreads / 64, kPfMaxC4 = 1024;
template <int NQ>  // weight quads per lane: C <= 256 NQ
__global__ void __launch_bounds__(kPfThreads) pool_fc_kernel(const float *x, const float *w, const float *bias,
                                                             float *out, long ldo, int P, int C, int F, int act,
                                                             float lo, float hi) {
    __shared__ float4 part_sum[kPfThreads];  // parts x C4 <= 1024 quads
    __shared__ float4 pooled[kPfMaxC4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = blockIdx.y;
    const int f = blockIdx.x * kPfOut + wave;
    const int C4 = C >> 2;
    constexpr unsigned OOB = 0x80000000u;

    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void *)w, (short)0, (int)((long)F * C * 4), 0x00020000);
    float4 wq[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
        const int q = lane + 64 * j;
        const unsigned o = f < F && q < C4 ? (unsigned)(((long)f * C + 4 * q) * 4) : OOB;
        wq[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, 0));
    }
    const float b = bias && f < F ? bias[f] : 0.0f;

    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(x + (long)i * P * C), (short)0, (int)((long)P * C * 4), 0x00020000);
    const int parts = kPfThreads / C4;
    const int part = tid / C4, q = tid - part * C4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (part < parts) {
        for (int p0 = part; p0 < P; p0 += 8 * parts) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int p = p0 + u * parts;
                const unsigned o = p < P ? (unsigned)(((long)p * C4 + q) * 16) : OOB;
                v[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0));
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                s.x += v[u].x;
                s.y += v[u].y;
                s.z += v[u].z;
                s.w += v[u].w;
            }
        }
        part_sum[part * C4 + q] = s;
    }
    __syncthreads();
    const float inv = 1.0f / (float)P;
    for (int e = tid; e < C4; e += kPfThreads) {
        float4 t = part_sum[e];
        for (int k = 1; k < parts; ++k) {
            const float4 u = part_sum[k * C4 + e];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
        pooled[e] = make_float4(t.x * inv, t.y * inv, t.z * inv, t.w * inv);
    }
    __syncthreads();

    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
        const int qq = lane + 64 * j;
        if (qq < C4) {
            const float4 pv = pooled[qq];
            acc = fmaf(wq[j].x, pv.x, acc);
            acc = fmaf(wq[j].y, pv.y, acc);
            acc = fmaf(wq[j].z, pv.z, acc);
            acc = fmaf(wq[j].w, pv.w, acc);
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
    if (lane == 0 && f < F) out[(long)i * ldo + f] = apply_act(acc + b, act, lo, hi);
}

}  // namespace mgc

using namespace mgc;

extern "C" void mgc_hip_gather_layer_norm(mgc_hip_exec *x, const mgc_hip_gather_ln_args *a) {
    if (a && a->rows <= 0) return;
    const bool ok = a && a->table && a->idx && a->out && a->dim > 0 && a->cols >= 4 && a->cols % 4 == 0 &&
                    a->cols <= 1024 && (a->idx_dtype == MGC_I64 || a->idx_dtype == MGC_I32) &&
                    (!a->addend || a->add_rows >= 1) &&
                    ((uintptr_t)a->table & 15) == 0 && ((uintptr_t)a->out & 15) == 0 &&
                    ((uintptr_t)a->addend & 15) == 0 && ((uintptr_t)a->scale & 15) == 0 &&
                    ((uintptr_t)a->bias & 15) == 0 && ((uintptr_t)a->sum & 15) == 0 && a->rows < (1L << 32);
    if (!ok) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_gather_layer_norm: shape, index type or alignment outside its limits",
                  hipErrorInvalidValue);
        return;
    }
    const long blocks = (a->rows + 3) / 4;  // four rows (one per wave) per workgroup
    MGC_LAUNCH(x, gather_add_layer_norm_rows, dim3((unsigned)blocks), dim3(256), 0, a->rows, a->cols / 4,
               (const float4 *)a->table, a->dim, a->idx, a->idx_dtype, (const float4 *)a->addend, a->add_rows,
               (const float4 *)a->scale, (const float4 *)a->bias, a->eps, (float4 *)a->out, (float4 *)a->sum,
               x->flag);
}

extern "C" int mgc_hip_pool_fc_supported(int N, int P, int C, int F) {
    return N >= 1 && N <= 65535 && P >= 1 && F >= 1 && C >= 4 && C % 4 == 0 && C / 4 <= kPfMaxC4 &&
           (long)F * C * 4 < 0x7fffffffL && (long)P * C * 4 < 0x7fffffffL;
}

extern "C" void mgc_hip_pool_fc(mgc_hip_exec *x, const mgc_hip_pool_fc_args *a) {
    if (a && (a->N <= 0 || a->F <= 0)) return;
    if (!a || !mgc_hip_pool_fc_supported(a->N, a->P, a->C, a->F) || !a->x || !a->w || !a->out ||
        ((uintptr_t)a->x & 15) != 0 || ((uintptr_t)a->w & 15) != 0 || a->ldo < a->F) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_pool_fc: shape, alignment or output stride outside its limits", hipErrorInvalidValue);
        return;
    }
    const int nq = (a->C / 4 + 63) / 64;
    const dim3 grid((unsigned)((a->F + kPfOut - 1) / kPfOut), (unsigned)a->N);
    const dim3 block(kPfThreads);
    using PoolFcKernel = void (*)(const float *, const float *, const float *, float *, long, int, int, int, int,
                                  float, float);
    const PoolFcKernel kern = nq <= 2   ? &pool_fc_kernel<2>
                              : nq <= 4 ? &pool_fc_kernel<4>
                              : nq <= 8 ? &pool_fc_kernel<8>
                                        : &pool_fc_kernel<16>;
    MGC_LAUNCH(x, kern, grid, block, 0, a->x, a->w, a->bias, a->out, a->ldo, a->P, a->C, a->F, a->act, a->lo, a->hi);
}

extern "C" void mgc_hip_reduce_mid(mgc_hip_exec *x, int is_max, long outer, long n, long inner,
                                   const float *in, float *out) {
    if (outer <= 0 || inner <= 0) return;
    if (inner == 1 && n >= 64) {
        MGC_LAUNCH(x, reduce_mid_rows, dim3(blocks_for(outer * 64, 256, 8192)), dim3(256), 0,
                   is_max, outer, n, in, out);
    } else if (inner % 4 == 0 && outer <= 65535 && n < 0x7fffffffL && inner < 0x7fffffffL &&
               (((uintptr_t)in | (uintptr_t)out) & 15) == 0) {
        const int inner4 = (int)(inner / 4);
        if (n >= 32) {
            MGC_LAUNCH(x, reduce_mid_vec4<16>, dim3((unsigned)((inner4 + 15) / 16), (unsigned)outer), dim3(256),
                       0, is_max, (int)n, inner4, (const float4 *)in, (float4 *)out);
        } else {
            MGC_LAUNCH(x, reduce_mid_vec4<64>, dim3((unsigned)((inner4 + 63) / 64), (unsigned)outer), dim3(256),
                       0, is_max, (int)n, inner4, (const float4 *)in, (float4 *)out);
        }
    } else {
        MGC_LAUNCH(x, reduce_mid_strided, dim3(blocks_for(outer * inner, 256, 8192)), dim3(256),
                   0, is_max, outer, n, inner, in, out);
    }
}

extern "C" void mgc_hip_reduce(mgc_hip_exec *x, int kind, int dtype, long outer, long n,
                               long inner, const void *in, void *out) {
    if (outer <= 0 || inner <= 0 || n <= 0) return;
    dim3 grid(blocks_for(outer * inner, 256, 8192));
    switch (dtype) {
    case MGC_F32:
        if (kind == 2 || kind == 3)
            MGC_LAUNCH(x, (reduce_generic<float, float>), grid, dim3(256), 0, kind, outer, n,
                       inner, (const float *)in, (float *)out);
        else
            MGC_LAUNCH(x, (reduce_generic<float, double>), grid, dim3(256), 0, kind, outer, n,
                       inner, (const float *)in, (float *)out);
        break;
    case MGC_F64:
        MGC_LAUNCH(x, (reduce_generic<double, double>), grid, dim3(256), 0, kind, outer, n,
                   inner, (const double *)in, (double *)out);
        break;
    case MGC_I64:
        MGC_LAUNCH(x, (reduce_generic<long long, long long>), grid, dim3(256), 0, kind, outer, n,
                   inner, (const long long *)in, (long long *)out);
        break;
    case MGC_I32:
        MGC_LAUNCH(x, (reduce_generic<int, long long>), grid, dim3(256), 0, kind, outer, n,
                   inner, (const int *)in, (int *)out);
        break;
    default:
        mgc::set_error("mgc_hip_reduce: unsupported dtype", hipErrorInvalidValue);
        break;
    }
}

extern "C" void mgc_hip_argmax(mgc_hip_exec *x, int dtype, long outer, long n, long inner,
                               const void *in, int64_t *out) {
    if (outer <= 0 || inner <= 0 || n <= 0) return;
    dim3 grid(blocks_for(outer * inner, 256, 8192));
    switch (dtype) {
    case MGC_F32:
        MGC_LAUNCH(x, argmax_kernel<float>, grid, dim3(256), 0, outer, n, inner,
                   (const float *)in, (long long *)out);
        break;
    case MGC_F64:
        MGC_LAUNCH(x, argmax_kernel<double>, grid, dim3(256), 0, outer, n, inner,
                   (const double *)in, (long long *)out);
        break;
    case MGC_I64:
        MGC_LAUNCH(x, argmax_kernel<long long>, grid, dim3(256), 0, outer, n, inner,
                   (const long long *)in, (long long *)out);
        break;
    case MGC_I32:
        MGC_LAUNCH(x, argmax_kernel<int>, grid, dim3(256), 0, outer, n, inner, (const int *)in,
                   (long long *)out);
        break;
    default:
        mgc::set_error("mgc_hip_argmax: unsupported dtype", hipErrorInvalidValue);
        break;
    }
}

extern "C" void mgc_hip_softmax(mgc_hip_exec *x, long outer, long n, long inner, const float *in,
                                float *out, int log_softmax) {
    if (outer <= 0 || inner <= 0 || n <= 0) return;
    if (inner == 1) {
        MGC_LAUNCH(x, softmax_rows, dim3(blocks_for(outer * 64, 256, 16384)), dim3(256), 0, outer,
                   n, in, out, log_softmax);
    } else {
        MGC_LAUNCH(x, softmax_strided, dim3(blocks_for(outer * inner, 256, 8192)), dim3(256), 0,
                   outer, n, inner, in, out, log_softmax);
    }
}

extern "C" void mgc_hip_layer_norm(mgc_hip_exec *x, long rows, long cols, const float *in,
                                   const float *scale, const float *bias, float eps, float *out) {
    if (rows <= 0 || cols <= 0) return;
    const bool vec = cols % 4 == 0 && cols <= 1024 && rows < (1L << 25) &&
                     (((uintptr_t)in | (uintptr_t)out | (uintptr_t)scale | (uintptr_t)bias) & 15) == 0;
    if (vec) {
        MGC_LAUNCH(x, layer_norm_rows_vec4, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (int)rows,
                   (int)(cols / 4), (const float4 *)in, (const float4 *)scale, (const float4 *)bias, eps,
                   (float4 *)out);
        return;
    }
    MGC_LAUNCH(x, layer_norm_rows, dim3(blocks_for(rows * 64, 256, 16384)), dim3(256), 0, rows,
               cols, in, scale, bias, eps, out);
}

extern "C" void mgc_hip_pool(mgc_hip_exec *x, int nhwc, int is_max, int N, int H, int W, int C,
                             int KH, int KW, int SH, int SW, int DH, int DW, int PT, int PL,
                             int PB, int PR, int OH, int OW, int count_include_pad,
                             const float *in, float *out) {
    PoolGeo g{N, H, W, C, KH, KW, SH, SW, DH, DW, PT, PL, PB, PR, OH, OW, count_include_pad,
              is_max};
    long total = (long)N * OH * OW * C;
    if (total <= 0) return;
    dim3 grid(blocks_for(total, 256, 16384));
    const bool vec = nhwc && C % 4 == 0 && total < 0x7fffffffL && (long)N * H * W * C < 0x7fffffffL &&
                     (((uintptr_t)in | (uintptr_t)out) & 15) == 0;
    if (vec) {
        const int quads = (int)(total / 4);
        auto kern = KH == 3 && KW == 3 ? pool_nhwc_vec4<3> : pool_nhwc_vec4<0>;
        MGC_LAUNCH(x, kern, dim3(blocks_for(quads, 256, 16384)), dim3(256), 0, g,
                   make_fastdiv((unsigned)(C / 4)), make_fastdiv((unsigned)OW), make_fastdiv((unsigned)OH),
                   quads, in, out);
    } else if (nhwc) {
        MGC_LAUNCH(x, pool_nhwc, grid, dim3(256), 0, g, in, out);
    } else {
        MGC_LAUNCH(x, pool_nchw, grid, dim3(256), 0, g, in, out);
    }
}

// The stride-1 3x3 depthwise form: on wide rows (OW >= 28) the preloading kernel with two
// outputs per thread (every input, weight and residual load issued before the first FMA), on
// narrow rows the row-by-row column kernel. MobileNetV2's stride-1 layers at batch 32, eager
// hipEvent timing of 50 launches, against the row-by-row kernel with four outputs per thread:
// 56 x 56 x 144 16.9 vs 28.1 us (85% of 8 TB/s), 28 x 28 x 192 8.2 vs 12.2 us; the preloading
// kernel on the 14 x 14 and 7 x 7 layers was 0-8% slower than the two-output column kernel.
// Large launches whose input does not stay in the caches keep the row-by-row kernel with four
// outputs per thread (fewer refetches of the shared input columns): 112 x 112 x 144 at batch 32
// (231 MB of input) 121 us against 198 us with the preloading kernel.
static bool dw3_preload_s1(int OW, long in_bytes) { return OW >= 28 && in_bytes <= (64L << 20); }
static int dw3_tile_s1(int OW) { return OW >= 28 ? 4 : 2; }

// The LDS-tiled 3x3 kernel (equal strides) for launches of at most 2^18 output quads: there a
// workgroup's three loads per thread, all issued before the first is used, beat the per-thread
// column kernel (MobileNetV2 at batch 1: 0.404 vs 0.428 ms per forward). On large launches it
// measured slower (the 112 x 112 x 144 s1 layer of 32 images at 32% of HBM peak instead of 47%:
// its 128-byte channel slices of 576-byte pixels straddle cache lines and the tile does not
// overlap its loads with its arithmetic), so those take the preloading or row-streaming kernel.
static bool dw3_lds(int N, int OH, int OW, int C) {
    return (long)N * OH * OW * (C / 4) <= (1L << 18);
}

extern "C" void mgc_hip_depthwise(mgc_hip_exec *x, int nhwc, int N, int H, int W, int C, int KH,
                                  int KW, int SH, int SW, int DH, int DW, int PT, int PL, int OH,
                                  int OW, const float *in, const float *w, const float *bias,
                                  const float *res, int act, float lo, float hi, float *out) {
    DwGeo g{N, H, W, C, KH, KW, SH, SW, DH, DW, PT, PL, OH, OW, act, lo, hi};
    long total = (long)N * OH * OW * C;
    if (total <= 0) return;
    if (nhwc) {
        bool vec = C % 4 == 0 && total / 4 < 0x7fffffffL && (long)N * H * W * C < 0x7fffffffL &&
                   (((uintptr_t)in | (uintptr_t)w | (uintptr_t)out | (uintptr_t)bias | (uintptr_t)res) & 15) == 0;
        const bool k3 = KH == 3 && KW == 3 && DH == 1 && DW == 1 && (SW == 1 || SW == 2);
        const int tiles_w = (OW + 7) / 8, tiles_h = (OH + 7) / 8, cgroups = (C / 4 + 7) / 8;
        const long blocks = (long)N * tiles_h * tiles_w * cgroups;
        const bool lds = vec && k3 && SH == SW && dw3_lds(N, OH, OW, C) && blocks < 0x7fffffffL;
        if (lds) {
            auto kern = SW == 2 ? depthwise3x3_nhwc_lds<2> : depthwise3x3_nhwc_lds<1>;
            MGC_LAUNCH(x, kern, dim3((unsigned)blocks), dim3(256), 0, g, tiles_w, tiles_h, cgroups, in, w, bias,
                       res, out);
        } else if (vec && k3 && SH == 1 && SW == 1 && PT <= 1 && PL <= 1 &&
                   !dw3_preload_s1(OW, (long)N * H * W * C * 4)) {
            // the row-streaming kernel where the column kernels would run (inputs over 64 MB,
            // narrow rows): 32 x 112 x 112 x 144 in 98 us against 128 us (hipEvent timing, one
            // box); one round of two workgroups per CU, each walking OH / 4 rows or more
            // channel slices of at most kDwRowsCQ quads, as even as they go; strips of
            // 4 * floor(256 / cq) columns
            const int cgr = (C / 4 + kDwRowsCQ - 1) / kDwRowsCQ;
            const int cq = (C / 4 + cgr - 1) / cgr;
            const int tw = 4 * (256 / cq);
            const int strips = (OW + tw - 1) / tw;
            const long base = (long)N * strips * cgr;
            long chunks = (512 + base - 1) / base;
            if (chunks > (OH + 3) / 4) chunks = (OH + 3) / 4;
            if (chunks < 1) chunks = 1;
            const int rows_per = (int)((OH + chunks - 1) / chunks);
            chunks = (OH + rows_per - 1) / rows_per;
            MGC_LAUNCH(x, depthwise3x3_nhwc_rows, dim3((unsigned)(base * chunks)), dim3(256), 0, g, strips, cgr, cq,
                       (int)chunks, rows_per, in, w, bias, res, out);
        } else if (vec && k3) {
            const bool pre = SW == 2 || dw3_preload_s1(OW, (long)N * H * W * C * 4);
            const int tile = pre ? 2 : dw3_tile_s1(OW);
            const int owb = (OW + tile - 1) / tile;
            const int quads = (int)((long)N * OH * owb * (C / 4));
            auto kern = SW == 2 ? depthwise3x3_nhwc_preload<2, 2>
                        : pre   ? depthwise3x3_nhwc_preload<1, 2>
                        : tile == 4 ? depthwise3x3_nhwc_vec4<1, 4>
                                    : depthwise3x3_nhwc_vec4<1, 2>;
            MGC_LAUNCH(x, kern, dim3(blocks_for(quads, 256, 16384)), dim3(256), 0, g,
                       make_fastdiv((unsigned)(C / 4)), make_fastdiv((unsigned)owb), make_fastdiv((unsigned)OH),
                       quads, in, w, bias, res, out);
        } else if (vec)
            MGC_LAUNCH(x, depthwise_nhwc_vec4, dim3(blocks_for(total / 4, 256, 16384)), dim3(256),
                       0, g, make_fastdiv((unsigned)(C / 4)), make_fastdiv((unsigned)OW),
                       make_fastdiv((unsigned)OH), (int)(total / 4), in, w, bias, res, out);
        else
            MGC_LAUNCH(x, depthwise_nhwc, dim3(blocks_for(total, 256, 16384)), dim3(256), 0, g, in,
                       w, bias, res, out);
    } else {
        MGC_LAUNCH(x, depthwise_nchw, dim3(blocks_for(total, 256, 16384)), dim3(256), 0, g, in, w,
                   bias, res, out);
    }
}
