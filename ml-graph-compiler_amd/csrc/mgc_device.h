// Internal header of libmgc_hip.so: execution context, launch helpers and device math.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mgc_hip.h"

// One model's execution context (opaque to generated code).
struct mgc_hip_exec {
    hipStream_t stream;
    int *flag;          // device int: 1 after an out-of-range Gather index
    int profiling;      // 1 while an eager profiled pass runs
    int n_nodes;
    hipEvent_t *ev_begin;
    hipEvent_t *ev_end;
    int launch_error;   // first launch failure seen since the last check (hipError_t)
};

namespace mgc {

// Record the first launch error of a pass; the runtime reports it as MGC_ERR_HIP.
void note_launch(mgc_hip_exec *x);
void set_error(const char *where, hipError_t err);

inline unsigned blocks_for(long n, int threads, long cap = 1L << 20) {
    long b = (n + threads - 1) / threads;
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return (unsigned)b;
}

// Division by a launch-constant divisor d (1 <= d < 2^31) for numerators 0 <= n < 2^31:
// q = (umulhi(n, m) + n) >> s with s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1
// (Granlund and Montgomery, "Division by invariant integers using multiplication", 1994).
struct FastDiv {
    unsigned d, m, s;
};

inline FastDiv make_fastdiv(unsigned d) {
    FastDiv f;
    f.d = d ? d : 1;
    f.s = 0;
    while ((1u << f.s) < f.d) ++f.s;
    f.m = (unsigned)((((unsigned long long)1 << 32) * (((unsigned long long)1 << f.s) - f.d)) / f.d + 1);
    return f;
}

__device__ __forceinline__ int fdiv(int n, const FastDiv &f) {
    return (int)((__umulhi((unsigned)n, f.m) + (unsigned)n) >> f.s);
}

// Workgroup ids of a 1-D grid are dealt round-robin to the 8 XCDs, each with its own L2. This
// renumbering (a permutation of 0..gridDim.x-1) gives XCD x a contiguous range of logical
// blocks, so neighbouring blocks that read overlapping input rows share one L2 instead of each
// XCD fetching the rows from HBM again.
__device__ __forceinline__ int xcd_block() {
    const int nb = gridDim.x, b = blockIdx.x;
    const int per = nb >> 3, rem = nb & 7, x = b & 7, i = b >> 3;
    return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

// ------------------------------------------------------------------------------------------
// device math. exp/log/sqrt/tanh come from the HIP device library; erf uses the rational
// approximation the reference's interpreter and C runtime share (ops.py:201-229,
// mgc_runtime.h:59-78), so GELU matches them to float rounding.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ float erf_rational(float x) {
    x = fminf(fmaxf(x, -4.0f), 4.0f);
    float x2 = x * x;
    float p = -2.72614225801306e-10f;
    p = fmaf(p, x2, 2.77068142495902e-08f);
    p = fmaf(p, x2, -2.10102402082508e-06f);
    p = fmaf(p, x2, -5.69250639462346e-05f);
    p = fmaf(p, x2, -7.34990630326855e-04f);
    p = fmaf(p, x2, -2.95459980854025e-03f);
    p = fmaf(p, x2, -1.60960333262415e-02f);
    float q = -1.45660718464996e-05f;
    q = fmaf(q, x2, -2.13374055278905e-04f);
    q = fmaf(q, x2, -1.68282697438203e-03f);
    q = fmaf(q, x2, -7.37332916720468e-03f);
    q = fmaf(q, x2, -1.42647390514189e-02f);
    return x * p / q;
}

__device__ __forceinline__ float tanh_f(float x) { return tanhf(x); }

__device__ __forceinline__ float sigmoid_f(float x) { return 0.5f + 0.5f * tanhf(0.5f * x); }

__device__ __forceinline__ float gelu_erf_f(float x) {
    return 0.5f * x * (1.0f + erf_rational(x * 0.70710678118654752f));
}

__device__ __forceinline__ float gelu_tanh_f(float x) {
    return 0.5f * x * (1.0f + tanhf(0.79788456080286536f * (x + 0.044715f * x * x * x)));
}

__device__ __forceinline__ float apply_act(float v, int act, float lo, float hi) {
    switch (act) {
    case MGC_ACT_RELU: return v > 0.0f ? v : 0.0f;
    case MGC_ACT_CLIP: return fminf(fmaxf(v, lo), hi);
    case MGC_ACT_GELU: return gelu_erf_f(v);
    case MGC_ACT_GELU_TANH: return gelu_tanh_f(v);
    case MGC_ACT_TANH: return tanh_f(v);
    case MGC_ACT_SIGMOID: return sigmoid_f(v);
    default: return v;
    }
}

// Wave (64 lanes) reductions through DPP/permute-free shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// The LayerNorm's per-column scale and bias quads one lane applies (column quad lane + 64 j),
// read before the row's mean is known so that their latency overlaps the row's own loads and
// reductions; has_scale / has_bias record whether the operands exist.
struct LnAffine {
    float4 s[4], b[4];
    bool has_scale, has_bias;
};

__device__ __forceinline__ LnAffine ln_affine_load(int lane, int cols4, const float4 *scale, const float4 *bias) {
    LnAffine a;
    a.has_scale = scale != nullptr;
    a.has_bias = bias != nullptr;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = lane + 64 * j;
        const bool ok = k < cols4;
        a.s[j] = a.has_scale && ok ? scale[k] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        a.b[j] = a.has_bias && ok ? bias[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    return a;
}

// LayerNorm of one row held by a wavefront as up to four float4 per lane (v[j] is column quad
// lane + 64 j, zero where that is >= cols4): two-pass mean and variance in float, then
// (x - mean) / sqrt(var + eps) * scale + bias written to dst (the scale and bias steps are
// skipped where the operand is absent). Every lane of the wave must call it. Shared by the
// LayerNorm kernel and the split-K reduction that ends in a LayerNorm, so both round
// identically.
__device__ __forceinline__ void layer_norm_row_vec4(const float4 (&v)[4], int lane, int cols4, const LnAffine &aff,
                                                    float eps, float4 *dst) {
    const float cols = (float)(cols4 * 4);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) sum += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    const float mean = wave_sum(sum) / cols;
    float var = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (lane + 64 * j < cols4) {
            const float dx = v[j].x - mean, dy = v[j].y - mean, dz = v[j].z - mean, dw = v[j].w - mean;
            var += (dx * dx + dy * dy) + (dz * dz + dw * dw);
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(var) / cols + eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = lane + 64 * j;
        if (k < cols4) {
            float4 y = make_float4((v[j].x - mean) * inv, (v[j].y - mean) * inv, (v[j].z - mean) * inv,
                                   (v[j].w - mean) * inv);
            if (aff.has_scale) {
                y.x *= aff.s[j].x;
                y.y *= aff.s[j].y;
                y.z *= aff.s[j].z;
                y.w *= aff.s[j].w;
            }
            if (aff.has_bias) {
                y.x += aff.b[j].x;
                y.y += aff.b[j].y;
                y.z += aff.b[j].z;
                y.w += aff.b[j].w;
            }
            dst[k] = y;
        }
    }
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

}  // namespace mgc

#define MGC_LAUNCH(x, kernel, grid, block, shmem, ...)                                         \
    do {                                                                                       \
        hipLaunchKernelGGL(kernel, grid, block, shmem, (x)->stream, __VA_ARGS__);              \
        mgc::note_launch(x);                                                                   \
    } while (0)
