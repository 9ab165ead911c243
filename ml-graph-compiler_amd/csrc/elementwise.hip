// Elementwise programs, strided copies, fills, gathers and ranges.
//
// The reference's C backend emits one broadcast-strided loop nest per elementwise node or
// FusedElementwise program (src/ml_graph_compiler/codegen/c.py:360-529) and identity-body loop
// nests for the copy family (c.py:558-660). Here those bodies are data: the emitter encodes the
// program (leaf operands with element strides over the collapsed output dims, then a list of
// typed instructions) into mgc_hip_ew_args, and one grid-stride kernel evaluates it per element.
// Every branch on the program is uniform across the wavefront (it depends only on kernel
// arguments), so it runs on the scalar unit; the vector unit only does the arithmetic, loads
// and stores. Registers hold 64-bit patterns: float32 bits, float64 bits, or sign-extended
// integers, and every integer result is narrowed to its output dtype the way numpy's _keep does.
#include "mgc_device.h"

namespace mgc {

__device__ __forceinline__ float rf(uint64_t v) { return __uint_as_float((uint32_t)v); }
__device__ __forceinline__ uint64_t wf(float f) { return (uint64_t)__float_as_uint(f); }
__device__ __forceinline__ double rd(uint64_t v) { return __longlong_as_double((long long)v); }
__device__ __forceinline__ uint64_t wd(double d) { return (uint64_t)__double_as_longlong(d); }

__device__ __forceinline__ bool is_float(int dt) { return dt == MGC_F32 || dt == MGC_F64; }

__device__ __forceinline__ uint64_t load_elem(const void *p, int dt, long i) {
    switch (dt) {
    case MGC_F32: return wf(static_cast<const float *>(p)[i]);
    case MGC_F64: return wd(static_cast<const double *>(p)[i]);
    case MGC_I64: return (uint64_t) static_cast<const long long *>(p)[i];
    case MGC_I32: return (uint64_t)(long long) static_cast<const int *>(p)[i];
    case MGC_I8: return (uint64_t)(long long) static_cast<const signed char *>(p)[i];
    case MGC_U8: return (uint64_t) static_cast<const unsigned char *>(p)[i];
    default: return static_cast<const unsigned char *>(p)[i] != 0 ? 1u : 0u;
    }
}

__device__ __forceinline__ void store_elem(void *p, int dt, long i, uint64_t v) {
    switch (dt) {
    case MGC_F32: static_cast<float *>(p)[i] = rf(v); break;
    case MGC_F64: static_cast<double *>(p)[i] = rd(v); break;
    case MGC_I64: static_cast<long long *>(p)[i] = (long long)v; break;
    case MGC_I32: static_cast<int *>(p)[i] = (int)(long long)v; break;
    case MGC_I8: static_cast<signed char *>(p)[i] = (signed char)(long long)v; break;
    case MGC_U8: static_cast<unsigned char *>(p)[i] = (unsigned char)(long long)v; break;
    default: static_cast<unsigned char *>(p)[i] = v != 0 ? 1 : 0; break;
    }
}

// Narrow an int64 result to the width of dtype (wrap-around like a numpy cast).
__device__ __forceinline__ uint64_t narrow(long long v, int dt) {
    switch (dt) {
    case MGC_I32: return (uint64_t)(long long)(int)v;
    case MGC_I8: return (uint64_t)(long long)(signed char)v;
    case MGC_U8: return (uint64_t)(unsigned char)v;
    case MGC_BOOL: return v != 0 ? 1u : 0u;
    default: return (uint64_t)v;
    }
}

// Convert a register of dtype `from` to dtype `to` (ONNX Cast; float -> int truncates).
__device__ __forceinline__ uint64_t cast_reg(uint64_t v, int from, int to) {
    if (from == to) return v;
    if (to == MGC_BOOL) {
        if (from == MGC_F32) return rf(v) != 0.0f;
        if (from == MGC_F64) return rd(v) != 0.0;
        return (long long)v != 0;
    }
    if (to == MGC_F32) {
        if (from == MGC_F64) return wf((float)rd(v));
        return wf((float)(long long)v);
    }
    if (to == MGC_F64) {
        if (from == MGC_F32) return wd((double)rf(v));
        return wd((double)(long long)v);
    }
    long long iv;
    if (from == MGC_F32)
        iv = (long long)rf(v);
    else if (from == MGC_F64)
        iv = (long long)rd(v);
    else
        iv = (long long)v;
    return narrow(iv, to);
}

__device__ __forceinline__ float f32_op(const mgc_hip_ew_instr &in, float a, float b, float c,
                                        bool has_b, bool has_c) {
    switch (in.op) {
    case MGC_EW_ADD: return a + b;
    case MGC_EW_SUB: return a - b;
    case MGC_EW_MUL: return a * b;
    case MGC_EW_DIV: return a / b;
    case MGC_EW_POW: return powf(a, b);
    case MGC_EW_MAX: return fmaxf(a, b);
    case MGC_EW_MIN: return fminf(a, b);
    case MGC_EW_RELU: return a > 0.0f ? a : 0.0f;
    case MGC_EW_SIGMOID: return sigmoid_f(a);
    case MGC_EW_TANH: return tanhf(a);
    case MGC_EW_ERF: return erf_rational(a);
    case MGC_EW_SQRT: return sqrtf(a);
    case MGC_EW_EXP: return expf(a);
    case MGC_EW_LOG: return logf(a);
    case MGC_EW_NEG: return -a;
    case MGC_EW_ABS: return fabsf(a);
    case MGC_EW_RECIPROCAL: return 1.0f / a;
    case MGC_EW_FLOOR: return floorf(a);
    case MGC_EW_CEIL: return ceilf(a);
    case MGC_EW_SIN: return sinf(a);
    case MGC_EW_COS: return cosf(a);
    case MGC_EW_SOFTPLUS: return a > 20.0f ? a : log1pf(expf(a));
    case MGC_EW_GELU: return gelu_erf_f(a);
    case MGC_EW_GELU_TANH: return gelu_tanh_f(a);
    case MGC_EW_LEAKY_RELU: return a >= 0.0f ? a : in.fa * a;
    case MGC_EW_HARD_SIGMOID: return fminf(fmaxf(in.fa * a + in.fb, 0.0f), 1.0f);
    case MGC_EW_CLIP: return fminf(fmaxf(a, has_b ? b : in.fa), has_c ? c : in.fb);
    default: return a;  // Identity
    }
}

__device__ __forceinline__ double f64_op(const mgc_hip_ew_instr &in, double a, double b,
                                         double c, bool has_b, bool has_c) {
    switch (in.op) {
    case MGC_EW_ADD: return a + b;
    case MGC_EW_SUB: return a - b;
    case MGC_EW_MUL: return a * b;
    case MGC_EW_DIV: return a / b;
    case MGC_EW_POW: return pow(a, b);
    case MGC_EW_MAX: return fmax(a, b);
    case MGC_EW_MIN: return fmin(a, b);
    case MGC_EW_RELU: return a > 0.0 ? a : 0.0;
    case MGC_EW_TANH: return tanh(a);
    case MGC_EW_SQRT: return sqrt(a);
    case MGC_EW_EXP: return exp(a);
    case MGC_EW_LOG: return log(a);
    case MGC_EW_NEG: return -a;
    case MGC_EW_ABS: return fabs(a);
    case MGC_EW_RECIPROCAL: return 1.0 / a;
    case MGC_EW_FLOOR: return floor(a);
    case MGC_EW_CEIL: return ceil(a);
    case MGC_EW_CLIP: return fmin(fmax(a, has_b ? b : (double)in.fa), has_c ? c : (double)in.fb);
    default: return a;
    }
}

__device__ __forceinline__ long long int_op(const mgc_hip_ew_instr &in, long long a, long long b,
                                            long long c, bool has_b, bool has_c) {
    switch (in.op) {
    case MGC_EW_ADD: return a + b;
    case MGC_EW_SUB: return a - b;
    case MGC_EW_MUL: return a * b;
    case MGC_EW_DIV: return b != 0 ? a / b : 0;
    case MGC_EW_MAX: return a > b ? a : b;
    case MGC_EW_MIN: return a < b ? a : b;
    case MGC_EW_NEG: return -a;
    case MGC_EW_ABS: return a < 0 ? -a : a;
    case MGC_EW_RELU: return a > 0 ? a : 0;
    case MGC_EW_CLIP: {
        long long v = a;
        if (has_b && v < b) v = b;
        if (has_c && v > c) v = c;
        return v;
    }
    default: return a;
    }
}

// Compare / logical ops produce bool from operands of dtype dt.
__device__ __forceinline__ bool cmp_op(int op, uint64_t a, uint64_t b, int dt) {
    if (op == MGC_EW_AND) return a != 0 && b != 0;
    if (op == MGC_EW_OR) return a != 0 || b != 0;
    if (op == MGC_EW_XOR) return (a != 0) != (b != 0);
    if (dt == MGC_F32) {
        float x = rf(a), y = rf(b);
        switch (op) {
        case MGC_EW_EQUAL: return x == y;
        case MGC_EW_LESS: return x < y;
        case MGC_EW_GREATER: return x > y;
        case MGC_EW_LESS_EQUAL: return x <= y;
        default: return x >= y;
        }
    }
    if (dt == MGC_F64) {
        double x = rd(a), y = rd(b);
        switch (op) {
        case MGC_EW_EQUAL: return x == y;
        case MGC_EW_LESS: return x < y;
        case MGC_EW_GREATER: return x > y;
        case MGC_EW_LESS_EQUAL: return x <= y;
        default: return x >= y;
        }
    }
    long long x = (long long)a, y = (long long)b;
    switch (op) {
    case MGC_EW_EQUAL: return x == y;
    case MGC_EW_LESS: return x < y;
    case MGC_EW_GREATER: return x > y;
    case MGC_EW_LESS_EQUAL: return x <= y;
    default: return x >= y;
    }
}

__device__ __forceinline__ uint64_t eval_instr(const mgc_hip_ew_instr &in, uint64_t a, uint64_t b,
                                               uint64_t c) {
    const bool has_b = in.args[1] >= 0, has_c = in.args[2] >= 0;
    switch (in.op) {
    case MGC_EW_EQUAL:
    case MGC_EW_LESS:
    case MGC_EW_GREATER:
    case MGC_EW_LESS_EQUAL:
    case MGC_EW_GREATER_EQUAL:
    case MGC_EW_AND:
    case MGC_EW_OR:
    case MGC_EW_XOR: return cmp_op(in.op, a, b, in.in_dtype) ? 1u : 0u;
    case MGC_EW_NOT: return a != 0 ? 0u : 1u;
    case MGC_EW_WHERE: return a != 0 ? b : c;
    case MGC_EW_CAST: return cast_reg(a, in.in_dtype, in.out_dtype);
    default: break;
    }
    if (in.in_dtype == MGC_F32) return wf(f32_op(in, rf(a), rf(b), rf(c), has_b, has_c));
    if (in.in_dtype == MGC_F64) return wd(f64_op(in, rd(a), rd(b), rd(c), has_b, has_c));
    return narrow(int_op(in, (long long)a, (long long)b, (long long)c, has_b, has_c), in.out_dtype);
}

#define MGC_NREG (MGC_EW_MAX_LEAVES + MGC_EW_MAX_INSTR)

// Register file access with constant indices only, so it stays in VGPRs. `idx` is uniform.
__device__ __forceinline__ uint64_t reg_get(const uint64_t (&R)[MGC_NREG], int idx) {
    switch (idx) {
#define MGC_CASE(i) case i: return R[i];
        MGC_CASE(0) MGC_CASE(1) MGC_CASE(2) MGC_CASE(3) MGC_CASE(4) MGC_CASE(5) MGC_CASE(6)
        MGC_CASE(7) MGC_CASE(8) MGC_CASE(9) MGC_CASE(10) MGC_CASE(11) MGC_CASE(12) MGC_CASE(13)
        MGC_CASE(14) MGC_CASE(15) MGC_CASE(16) MGC_CASE(17) MGC_CASE(18) MGC_CASE(19)
        MGC_CASE(20) MGC_CASE(21) MGC_CASE(22) MGC_CASE(23) MGC_CASE(24) MGC_CASE(25)
        MGC_CASE(26) MGC_CASE(27) MGC_CASE(28) MGC_CASE(29) MGC_CASE(30) MGC_CASE(31)
        MGC_CASE(32) MGC_CASE(33) MGC_CASE(34) MGC_CASE(35) MGC_CASE(36) MGC_CASE(37)
        MGC_CASE(38) MGC_CASE(39) MGC_CASE(40) MGC_CASE(41) MGC_CASE(42) MGC_CASE(43)
        MGC_CASE(44) MGC_CASE(45) MGC_CASE(46) MGC_CASE(47)
#undef MGC_CASE
    default: return 0;
    }
}

__device__ __forceinline__ void reg_set(uint64_t (&R)[MGC_NREG], int idx, uint64_t v) {
    switch (idx) {
#define MGC_CASE(i) case i: R[i] = v; break;
        MGC_CASE(16) MGC_CASE(17) MGC_CASE(18) MGC_CASE(19) MGC_CASE(20) MGC_CASE(21)
        MGC_CASE(22) MGC_CASE(23) MGC_CASE(24) MGC_CASE(25) MGC_CASE(26) MGC_CASE(27)
        MGC_CASE(28) MGC_CASE(29) MGC_CASE(30) MGC_CASE(31) MGC_CASE(32) MGC_CASE(33)
        MGC_CASE(34) MGC_CASE(35) MGC_CASE(36) MGC_CASE(37) MGC_CASE(38) MGC_CASE(39)
        MGC_CASE(40) MGC_CASE(41) MGC_CASE(42) MGC_CASE(43) MGC_CASE(44) MGC_CASE(45)
        MGC_CASE(46) MGC_CASE(47)
#undef MGC_CASE
    default: break;
    }
}

// ------------------------------------------------------------------------------------------
// float32 fast path: programs whose leaves, registers and output are all float32 (the common
// case: scaling, broadcast adds, activation chains). 32-bit indices with host-computed magic
// divisors, a float register file that the compiler keeps in VGPRs (uniform indices become
// v_movrels), and, when the innermost dim allows, four consecutive elements per thread with
// 16-byte loads and stores.
// ------------------------------------------------------------------------------------------
constexpr int EWF_RANK = 4, EWF_LEAVES = 8, EWF_INSTR = 8, EWF_REGS = EWF_LEAVES + EWF_INSTR;

struct EwF32Instr {
    int op, a, b, c;  // register indices (b, c: -1 when absent)
    float fa, fb;
};

struct EwF32Args {
    int rank;                  // collapsed output rank, innermost last
    int units;                 // threads' work items (elements, or groups of 4)
    int dims[EWF_RANK];        // innermost dim counted in work items
    FastDiv div[EWF_RANK];
    int n_leaves, n_instr;
    const float *leaf[EWF_LEAVES];
    int lst[EWF_LEAVES][EWF_RANK];  // element strides
    int leaf_bytes[EWF_LEAVES];     // bytes reachable from leaf[l] (0 past n_leaves)
    int leaf_quad[EWF_LEAVES];      // 1: the leaf's innermost stride is 1 (16-byte quads), 0: broadcast
    EwF32Instr ins[EWF_INSTR];
    float *out;
    int ost[EWF_RANK];
};

__device__ __forceinline__ float ewf_op(const EwF32Instr &in, float a, float b, float c) {
    switch (in.op) {
    case MGC_EW_ADD: return a + b;
    case MGC_EW_SUB: return a - b;
    case MGC_EW_MUL: return a * b;
    case MGC_EW_DIV: return a / b;
    case MGC_EW_POW: return powf(a, b);
    case MGC_EW_MAX: return fmaxf(a, b);
    case MGC_EW_MIN: return fminf(a, b);
    case MGC_EW_RELU: return a > 0.0f ? a : 0.0f;
    case MGC_EW_SIGMOID: return sigmoid_f(a);
    case MGC_EW_TANH: return tanhf(a);
    case MGC_EW_ERF: return erf_rational(a);
    case MGC_EW_SQRT: return sqrtf(a);
    case MGC_EW_EXP: return expf(a);
    case MGC_EW_LOG: return logf(a);
    case MGC_EW_NEG: return -a;
    case MGC_EW_ABS: return fabsf(a);
    case MGC_EW_RECIPROCAL: return 1.0f / a;
    case MGC_EW_FLOOR: return floorf(a);
    case MGC_EW_CEIL: return ceilf(a);
    case MGC_EW_SIN: return sinf(a);
    case MGC_EW_COS: return cosf(a);
    case MGC_EW_SOFTPLUS: return a > 20.0f ? a : log1pf(expf(a));
    case MGC_EW_GELU: return gelu_erf_f(a);
    case MGC_EW_GELU_TANH: return gelu_tanh_f(a);
    case MGC_EW_LEAKY_RELU: return a >= 0.0f ? a : in.fa * a;
    case MGC_EW_HARD_SIGMOID: return fminf(fmaxf(in.fa * a + in.fb, 0.0f), 1.0f);
    case MGC_EW_CLIP: return fminf(fmaxf(a, in.b >= 0 ? b : in.fa), in.c >= 0 ? c : in.fb);
    default: return a;  // Identity
    }
}

// NL leaves and NI instructions at most: the register file of a work item is NL + NI values
// per lane of the unit; small programs (one Add, one activation) take the small instantiation,
// whose few registers let twice as many waves, and so twice as many loads, be in flight.
template <bool VEC, int NL, int NI>
__global__ void __launch_bounds__(256) ew_f32_kernel(const EwF32Args e) {
    constexpr int W = VEC ? 4 : 1;
    constexpr int NR = NL + NI;
    for (int u = blockIdx.x * 256 + threadIdx.x; u < e.units; u += gridDim.x * 256) {
        int off[NL];
#pragma unroll
        for (int l = 0; l < NL; ++l) off[l] = 0;
        int ooff = 0;
        int rem = u;
#pragma unroll
        for (int d = EWF_RANK - 1; d >= 0; --d) {
            if (d < e.rank) {
                const int q = fdiv(rem, e.div[d]);
                int c = rem - q * e.dims[d];
                rem = q;
                if (d == e.rank - 1) c *= W;
                ooff += c * e.ost[d];
#pragma unroll
                for (int l = 0; l < NL; ++l) off[l] += c * e.lst[l][d];
            }
        }
        float R0[NR], R1[NR], R2[NR], R3[NR];
        if (VEC) {
            // one 16-byte buffer load per leaf, all issued before any is used: a broadcast leaf
            // takes element 0 of it, bytes past a leaf's extent (and every byte of an unused
            // leaf, whose extent is 0) read as zero
#pragma unroll
            for (int l = 0; l < NL; ++l) {
                const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                    (void *)e.leaf[l], (short)0, e.leaf_bytes[l], 0x00020000);
                const float4 v = __builtin_bit_cast(
                    float4, __builtin_amdgcn_raw_buffer_load_b128(rs, (unsigned)off[l] * 4u, 0, 0));
                const bool quad = e.leaf_quad[l] != 0;
                R0[l] = v.x;
                R1[l] = quad ? v.y : v.x;
                R2[l] = quad ? v.z : v.x;
                R3[l] = quad ? v.w : v.x;
            }
        } else {
#pragma unroll
            for (int l = 0; l < NL; ++l) {
                float v0 = 0.f;
                if (l < e.n_leaves) v0 = e.leaf[l][off[l]];
                R0[l] = R1[l] = R2[l] = R3[l] = v0;
            }
        }
#pragma unroll
        for (int r = NL; r < NR; ++r) R0[r] = R1[r] = R2[r] = R3[r] = 0.f;
        float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if (i >= e.n_instr) break;
            const EwF32Instr &in = e.ins[i];
            const int ia = in.a, ib = in.b >= 0 ? in.b : 0, ic = in.c >= 0 ? in.c : 0;
            o0 = ewf_op(in, R0[ia], R0[ib], R0[ic]);
            if (VEC) {
                o1 = ewf_op(in, R1[ia], R1[ib], R1[ic]);
                o2 = ewf_op(in, R2[ia], R2[ib], R2[ic]);
                o3 = ewf_op(in, R3[ia], R3[ib], R3[ic]);
            }
            R0[NL + i] = o0;
            R1[NL + i] = o1;
            R2[NL + i] = o2;
            R3[NL + i] = o3;
        }
        if (VEC) {
            *reinterpret_cast<float4 *>(e.out + ooff) = make_float4(o0, o1, o2, o3);
        } else {
            e.out[ooff] = o0;
        }
    }
}

// Merges adjacent dimensions that every operand walks contiguously (stride[d] ==
// stride[d + 1] * dims[d + 1] for the output and every leaf, broadcast leaves included), so the
// kernel splits each index over fewer dimensions: [16, 128, 768] + [1, 128, 768] becomes
// [16, 98304] + [1, 98304].
static void ew_coalesce(mgc_hip_ew_args &e) {
    int d = e.rank - 2;
    while (d >= 0) {
        bool ok = e.out_strides[d] == e.out_strides[d + 1] * e.dims[d + 1];
        for (int l = 0; l < e.n_leaves && ok; ++l)
            ok = e.leaf[l].strides[d] == e.leaf[l].strides[d + 1] * e.dims[d + 1];
        if (ok) {
            e.dims[d + 1] *= e.dims[d];
            for (int k = d; k + 1 < e.rank; ++k) {
                e.dims[k] = e.dims[k + 1];
                e.out_strides[k] = e.out_strides[k + 1];
                for (int l = 0; l < e.n_leaves; ++l) e.leaf[l].strides[k] = e.leaf[l].strides[k + 1];
            }
            --e.rank;
        }
        --d;
    }
}

// Builds the float32 fast-path arguments, or returns false when the program does not qualify.
// ``nl``: the leaf count of the kernel instantiation, where instruction results start.
static bool ew_f32_plan(const mgc_hip_ew_args *e, EwF32Args &f, bool &vec, int nl) {
    if (e->out_dtype != MGC_F32 || e->rank < 1 || e->rank > EWF_RANK || e->n_leaves < 1 ||
        e->n_leaves > EWF_LEAVES || e->n_instr < 1 || e->n_instr > EWF_INSTR)
        return false;
    long total = 1;
    for (int d = 0; d < e->rank; ++d) total *= e->dims[d];
    if (total <= 0 || total >= (1L << 31)) return false;
    for (int l = 0; l < e->n_leaves; ++l) {
        if (e->leaf[l].dtype != MGC_F32 || e->leaf[l].p == nullptr) return false;
        long ext = 1;
        for (int d = 0; d < e->rank; ++d) {
            if (e->leaf[l].strides[d] < 0) return false;
            ext += (e->dims[d] - 1) * e->leaf[l].strides[d];
        }
        if (ext >= (1L << 31)) return false;
        f.leaf_bytes[l] = ext * 4 < 0x7fffffffL ? (int)(ext * 4) : 0;
    }
    long oext = e->out_base + 1;
    for (int d = 0; d < e->rank; ++d) {
        if (e->out_strides[d] < 0) return false;
        oext += (e->dims[d] - 1) * e->out_strides[d];
    }
    if (e->out_base < 0 || oext >= (1L << 31)) return false;
    for (int i = 0; i < e->n_instr; ++i) {
        const mgc_hip_ew_instr &in = e->instr[i];
        if (in.in_dtype != MGC_F32 || in.out_dtype != MGC_F32) return false;
        switch (in.op) {
        case MGC_EW_EQUAL: case MGC_EW_LESS: case MGC_EW_GREATER: case MGC_EW_LESS_EQUAL:
        case MGC_EW_GREATER_EQUAL: case MGC_EW_AND: case MGC_EW_OR: case MGC_EW_XOR:
        case MGC_EW_WHERE: case MGC_EW_NOT: case MGC_EW_CAST:
            return false;
        default: break;
        }
        for (int k = 0; k < 3; ++k)
            if (in.args[k] >= e->n_leaves + i) return false;  // only earlier results
        if (in.args[0] < 0) return false;
    }
    const int r = e->rank - 1;
    vec = e->dims[r] % 4 == 0 && e->out_strides[r] == 1 && e->out_base % 4 == 0 &&
          (((uintptr_t)e->out) & 15) == 0;
    for (int d = 0; d < r && vec; ++d) vec = e->out_strides[d] % 4 == 0;
    for (int l = 0; l < e->n_leaves && vec; ++l) vec = f.leaf_bytes[l] > 0;  // buffer offsets are 32-bit
    for (int l = 0; l < e->n_leaves && vec; ++l) {
        const long st = e->leaf[l].strides[r];
        if (st == 1) {
            vec = (((uintptr_t)e->leaf[l].p) & 15) == 0;
            for (int d = 0; d < r && vec; ++d) vec = e->leaf[l].strides[d] % 4 == 0;
        } else {
            vec = st == 0;
        }
    }
    f.rank = e->rank;
    f.units = (int)(vec ? total / 4 : total);
    for (int d = 0; d < EWF_RANK; ++d) {
        const int dim = d < e->rank ? (int)e->dims[d] : 1;
        f.dims[d] = (vec && d == r) ? dim / 4 : dim;
        f.div[d] = make_fastdiv((unsigned)(f.dims[d] > 0 ? f.dims[d] : 1));
        f.ost[d] = d < e->rank ? (int)e->out_strides[d] : 0;
    }
    f.n_leaves = e->n_leaves;
    f.n_instr = e->n_instr;
    for (int l = 0; l < EWF_LEAVES; ++l) {
        f.leaf[l] = l < e->n_leaves ? static_cast<const float *>(e->leaf[l].p) : nullptr;
        if (l >= e->n_leaves) f.leaf_bytes[l] = 0;
        f.leaf_quad[l] = l < e->n_leaves && e->leaf[l].strides[r] == 1 ? 1 : 0;
        for (int d = 0; d < EWF_RANK; ++d)
            f.lst[l][d] = (l < e->n_leaves && d < e->rank) ? (int)e->leaf[l].strides[d] : 0;
    }
    // Registers: leaves 0 .. n_leaves - 1 keep their numbers; instruction i's result, register
    // MGC_EW_MAX_LEAVES + i in the generic encoding, becomes nl + i.
    auto remap = [&](int a) { return a < 0 ? -1 : (a < MGC_EW_MAX_LEAVES ? a : a - MGC_EW_MAX_LEAVES + nl); };
    for (int i = 0; i < EWF_INSTR; ++i) {
        EwF32Instr &o = f.ins[i];
        if (i < e->n_instr) {
            const mgc_hip_ew_instr &in = e->instr[i];
            o.op = in.op;
            o.a = remap(in.args[0]);
            o.b = remap(in.args[1]);
            o.c = remap(in.args[2]);
            o.fa = in.fa;
            o.fb = in.fb;
        } else {
            o.op = MGC_EW_IDENTITY;
            o.a = 0;
            o.b = o.c = -1;
            o.fa = o.fb = 0.f;
        }
    }
    f.out = static_cast<float *>(e->out) + e->out_base;
    return true;
}

__global__ void __launch_bounds__(256) ew_program_kernel(const mgc_hip_ew_args e) {
    long total = 1;
    for (int d = 0; d < e.rank; ++d) total *= e.dims[d];
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        long coord[MGC_EW_MAX_RANK];
        long rem = idx;
#pragma unroll
        for (int d = MGC_EW_MAX_RANK - 1; d >= 0; --d) {
            if (d < e.rank) {
                coord[d] = rem % e.dims[d];
                rem /= e.dims[d];
            } else {
                coord[d] = 0;
            }
        }
        uint64_t R[MGC_NREG];
#pragma unroll
        for (int l = 0; l < MGC_EW_MAX_LEAVES; ++l) {
            if (l < e.n_leaves && e.leaf[l].p) {
                long off = 0;
#pragma unroll
                for (int d = 0; d < MGC_EW_MAX_RANK; ++d)
                    if (d < e.rank) off += coord[d] * e.leaf[l].strides[d];
                R[l] = load_elem(e.leaf[l].p, e.leaf[l].dtype, off);
            } else {
                R[l] = 0;
            }
        }
#pragma unroll
        for (int i = MGC_EW_MAX_LEAVES; i < MGC_NREG; ++i) R[i] = 0;
        uint64_t last = 0;
        for (int i = 0; i < e.n_instr; ++i) {
            const mgc_hip_ew_instr &in = e.instr[i];
            uint64_t a = in.args[0] >= 0 ? reg_get(R, in.args[0]) : 0;
            uint64_t b = in.args[1] >= 0 ? reg_get(R, in.args[1]) : 0;
            uint64_t c = in.args[2] >= 0 ? reg_get(R, in.args[2]) : 0;
            last = eval_instr(in, a, b, c);
            reg_set(R, MGC_EW_MAX_LEAVES + i, last);
        }
        long ooff = e.out_base;
#pragma unroll
        for (int d = 0; d < MGC_EW_MAX_RANK; ++d)
            if (d < e.rank) ooff += coord[d] * e.out_strides[d];
        store_elem(e.out, e.out_dtype, ooff, last);
    }
}

// N-d strided copy with optional per-dim modulus (Tile). T is the moved unit.
template <typename T>
__global__ void __launch_bounds__(256) copy_kernel(const mgc_hip_copy_args c) {
    long total = 1;
    for (int d = 0; d < c.rank; ++d) total *= c.dims[d];
    const T *src = static_cast<const T *>(c.in);
    T *dst = static_cast<T *>(c.out);
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        long rem = idx, io = c.in_base, oo = c.out_base;
#pragma unroll
        for (int d = MGC_EW_MAX_RANK - 1; d >= 0; --d) {
            if (d < c.rank) {
                long q = rem / c.dims[d];
                long i = rem - q * c.dims[d];
                rem = q;
                oo += i * c.out_strides[d];
                io += (c.in_mod[d] ? i % c.in_mod[d] : i) * c.in_strides[d];
            }
        }
        dst[oo] = src[io];
    }
}

// A copy that moves the input's contiguous dim p to a strided output position while the
// output's contiguous dim q reads the input with a stride (a transpose of p and q): 64 x 64
// tiles through LDS, read with consecutive lanes along p and written with consecutive lanes
// along q, so both sides are coalesced (the element-wise copy would touch one element per
// 64-byte line on one side). blockIdx.z enumerates the other (batch) dims, at most two.
struct TransposeGeo {
    int np, nq;               // extents of p (input-contiguous) and q (output-contiguous)
    long in_q, out_p;         // the non-unit strides: input along q, output along p
    int nb0, nb1;             // batch extents (nb0 outermost)
    long in_b0, in_b1, out_b0, out_b1;
    long in_base, out_base;
};

template <typename T>
__global__ void __launch_bounds__(256) transpose_tiled_kernel(const TransposeGeo g, const T *in, T *out) {
    __shared__ T tile[64][65];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int q0 = blockIdx.x * 64, p0 = blockIdx.y * 64;
    const int b1 = blockIdx.z % g.nb1, b0 = blockIdx.z / g.nb1;
    const T *src = in + g.in_base + b0 * g.in_b0 + b1 * g.in_b1;
    T *dst = out + g.out_base + b0 * g.out_b0 + b1 * g.out_b1;
    const int p = p0 + tx;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int ql = ty + 4 * i, q = q0 + ql;
        if (p < g.np && q < g.nq) tile[ql][tx] = src[(long)q * g.in_q + p];
    }
    __syncthreads();
    const int q = q0 + tx;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int pl = ty + 4 * i, pp = p0 + pl;
        if (pp < g.np && q < g.nq) dst[(long)pp * g.out_p + q] = tile[tx][pl];
    }
}

// The same transpose with 16-byte global accesses (V = 16 / sizeof(T) elements per lane) when
// both extents, every stride and both bases are multiples of V and the pointers are 16-byte
// aligned: a wave moves 1 KB per load or store instruction instead of 256 bytes, which the
// address units, not HBM, limited. Lanes read V consecutive p of a q row into LDS, then V
// consecutive q of a p column out of it; with the 65-element row pitch both phases spread a
// wave's 64 lanes over all banks.
template <typename T>
__global__ void __launch_bounds__(256) transpose_tiled_vec_kernel(const TransposeGeo g, const T *in, T *out) {
    constexpr int V = 16 / sizeof(T), LP = 64 / V, RP = 256 / LP;
    __shared__ T tile[64][65];
    const int lx = threadIdx.x % LP, ly = threadIdx.x / LP;
    const int q0 = blockIdx.x * 64, p0 = blockIdx.y * 64;
    const int b1 = blockIdx.z % g.nb1, b0 = blockIdx.z / g.nb1;
    const T *src = in + g.in_base + b0 * g.in_b0 + b1 * g.in_b1;
    T *dst = out + g.out_base + b0 * g.out_b0 + b1 * g.out_b1;
    const int p = p0 + lx * V;
#pragma unroll
    for (int i = 0; i < 64 / RP; ++i) {
        const int ql = ly + RP * i, q = q0 + ql;
        if (p < g.np && q < g.nq) {
            const uint4 v = *reinterpret_cast<const uint4 *>(src + (long)q * g.in_q + p);
            const T *e = reinterpret_cast<const T *>(&v);
#pragma unroll
            for (int k = 0; k < V; ++k) tile[ql][lx * V + k] = e[k];
        }
    }
    __syncthreads();
    const int q = q0 + lx * V;
#pragma unroll
    for (int i = 0; i < 64 / RP; ++i) {
        const int pl = ly + RP * i, pp = p0 + pl;
        if (pp < g.np && q < g.nq) {
            uint4 v;
            T *e = reinterpret_cast<T *>(&v);
#pragma unroll
            for (int k = 0; k < V; ++k) e[k] = tile[lx * V + k][pl];
            *reinterpret_cast<uint4 *>(dst + (long)pp * g.out_p + q) = v;
        }
    }
}

// The tiled transpose applies when the output's innermost dim q is read with a stride while
// another dim p is the input's contiguous one, both at least 32 long, with no modulus and at
// most two other dims; fills g and the grid and returns true then.
static bool transpose_plan(const mgc_hip_copy_args &c, TransposeGeo &g, dim3 &grid) {
    const int r = c.rank;
    if (r < 2 || r > 4 || (c.elem_bytes != 4 && c.elem_bytes != 8)) return false;
    const int q = r - 1;
    if (c.out_strides[q] != 1 || c.in_strides[q] == 1) return false;
    int p = -1;
    for (int d = 0; d < r; ++d) {
        if (c.in_mod[d] != 0) return false;
        if (d != q && c.in_strides[d] == 1) p = d;
    }
    if (p < 0 || c.dims[p] < 32 || c.dims[q] < 32 || c.dims[p] > 0x7fffffff || c.dims[q] > 0x7fffffff)
        return false;
    int batch[2] = {-1, -1}, nb = 0;
    for (int d = 0; d < r; ++d)
        if (d != p && d != q) batch[nb++] = d;
    g.np = (int)c.dims[p];
    g.nq = (int)c.dims[q];
    g.in_q = c.in_strides[q];
    g.out_p = c.out_strides[p];
    g.nb0 = batch[0] >= 0 ? (int)c.dims[batch[0]] : 1;
    g.nb1 = batch[1] >= 0 ? (int)c.dims[batch[1]] : 1;
    g.in_b0 = batch[0] >= 0 ? c.in_strides[batch[0]] : 0;
    g.out_b0 = batch[0] >= 0 ? c.out_strides[batch[0]] : 0;
    g.in_b1 = batch[1] >= 0 ? c.in_strides[batch[1]] : 0;
    g.out_b1 = batch[1] >= 0 ? c.out_strides[batch[1]] : 0;
    g.in_base = c.in_base;
    g.out_base = c.out_base;
    const long nbatch = (long)g.nb0 * g.nb1;
    if (nbatch < 1 || nbatch > 65535) return false;
    grid = dim3((unsigned)((g.nq + 63) / 64), (unsigned)((g.np + 63) / 64), (unsigned)nbatch);
    return grid.y <= 65535;
}

// One thread per output pixel (b, i, j): two 8-byte reads per channel and row of the 2 x 2
// block (neighbouring threads read neighbouring pairs), C 16-byte writes of the pixel's 4 C
// values (neighbouring threads write neighbouring 16 C-byte groups).
__global__ void space_to_depth_kernel(int C, int H2, int W2, int total, FastDiv div_w2, FastDiv div_h2,
                                      const float *in, float *out) {
    const int H = 2 * H2, W = 2 * W2;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const int t = fdiv(idx, div_w2);
        const int j = idx - t * W2;
        const int b = fdiv(t, div_h2);
        const int i = t - b * H2;
        float v[32];
        const float *src = in + (long)b * C * H * W + (long)(2 * i) * W + 2 * j;
        for (int c = 0; c < C; ++c) {
#pragma unroll
            for (int dy = 0; dy < 2; ++dy) {
                const float2 pr = *reinterpret_cast<const float2 *>(src + (long)c * H * W + dy * W);
                v[(dy * 2) * C + c] = pr.x;
                v[(dy * 2 + 1) * C + c] = pr.y;
            }
        }
        float4 *dst = reinterpret_cast<float4 *>(out + (long)idx * 4 * C);
        for (int q = 0; q < C; ++q) dst[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    }
}

// The same for C <= 4, W % 4 == 0 and 16-byte aligned input: one thread per pair of
// neighbouring output pixels (b, i, 2 jp .. 2 jp + 1), whose 2 x 4 input block per channel is two
// 16-byte reads (neighbouring threads read neighbouring 16 bytes of a row). The pair's 8 C output
// values are contiguous and so are the 64 pairs of a wave, so the wave stages its 64 x 8 C values
// in LDS and writes them back as whole contiguous 1 KB rows (lane l writes 16 bytes at 16 l of
// each), instead of 16-byte pieces 32 C bytes apart. Each wave takes several 64-pair blocks in
// turn and requests the next block's input before it stages and stores the current one, so its
// reads of one block overlap its writes of the previous (one read round and one write round per
// launch otherwise, each waiting for the whole chip's).
template <int C>
__global__ void __launch_bounds__(256) space_to_depth_vec_kernel(int H2, int W4, int total, FastDiv div_w4,
                                                                 FastDiv div_h2, const float *in, float *out) {
    constexpr int PAIR = 8 * C;  // floats per pair of output pixels
    __shared__ __attribute__((aligned(16))) float stage[4][64 * PAIR];
    const int H = 2 * H2, W = 4 * W4;
    const int lane = threadIdx.x & 63;
    float *const buf = stage[threadIdx.x >> 6];
    const int step = gridDim.x * blockDim.x;
    // the 2 x 4 input block of every channel of the lane's pair in the wave's block at base
    auto load = [&](int base, float4 (&row)[C][2]) __attribute__((always_inline)) {
        const int idx = base + lane;
        if (idx < total) {
            const int t = fdiv(idx, div_w4);
            const int jp = idx - t * W4;
            const int b = fdiv(t, div_h2);
            const int i = t - b * H2;
            const float *src = in + (long)b * C * H * W + (long)(2 * i) * W + 4 * jp;
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int dy = 0; dy < 2; ++dy)
                    row[c][dy] = *reinterpret_cast<const float4 *>(src + (long)c * H * W + dy * W);
        }
    };
    // every lane of a wave runs the same trips (the bound is the wave's first pair)
    int base = blockIdx.x * blockDim.x + (threadIdx.x & ~63);
    float4 cur[C][2], nxt[C][2];
    if (base < total) load(base, cur);
    for (; base < total; base += step) {
        if (base + step < total) load(base + step, nxt);
        // output pixel q of the pair holds value (dy * 2 + dx) * C + c = input (c, dy, 2 q + dx)
        if (base + lane < total) {
            float *v = buf + lane * PAIR;
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int dy = 0; dy < 2; ++dy) {
                    v[(dy * 2) * C + c] = cur[c][dy].x;
                    v[(dy * 2 + 1) * C + c] = cur[c][dy].y;
                    v[4 * C + (dy * 2) * C + c] = cur[c][dy].z;
                    v[4 * C + (dy * 2 + 1) * C + c] = cur[c][dy].w;
                }
        }
        __builtin_amdgcn_wave_barrier();
        // the wave's pairs [base, base + n) are out[base * PAIR ...] contiguous
        const int n = min(64, total - base);
        const float4 *src4 = reinterpret_cast<const float4 *>(buf);
        float4 *dst4 = reinterpret_cast<float4 *>(out + (long)base * PAIR);
#pragma unroll
        for (int q = 0; q < 2 * C; ++q) {
            const int e = q * 64 + lane;  // 16-byte chunk of the wave's block
            if (e < n * 2 * C) dst4[e] = src4[e];
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int dy = 0; dy < 2; ++dy) cur[c][dy] = nxt[c][dy];
    }
}

template <typename T>
__global__ void fill_kernel(T *out, long n, T v) {
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n;
         i += (long)gridDim.x * blockDim.x)
        out[i] = v;
}

// One workgroup per (outer, t) row; the row is copied in 4-byte words when aligned.
__global__ void gather_kernel(const unsigned char *src, const void *idx, int idx_dtype,
                              long outer, long dim, long n, long inner_bytes, unsigned char *out,
                              int *flag) {
    for (long row = blockIdx.x; row < outer * n; row += gridDim.x) {
        const long o = row / n, t = row - (row / n) * n;
        long k = idx_dtype == MGC_I64 ? static_cast<const long long *>(idx)[t]
                                      : (long)static_cast<const int *>(idx)[t];
        if (k < 0) k += dim;
        if (k < 0 || k >= dim) {
            if (threadIdx.x == 0) *flag = 1;
            continue;
        }
        const unsigned char *s = src + (o * dim + k) * inner_bytes;
        unsigned char *d = out + (o * n + t) * inner_bytes;
        if ((inner_bytes & 3) == 0 && (((uintptr_t)s | (uintptr_t)d) & 3) == 0) {
            const long words = inner_bytes >> 2;
            for (long w = threadIdx.x; w < words; w += blockDim.x)
                reinterpret_cast<unsigned *>(d)[w] = reinterpret_cast<const unsigned *>(s)[w];
        } else {
            for (long b = threadIdx.x; b < inner_bytes; b += blockDim.x) d[b] = s[b];
        }
    }
}

// Rows of a multiple of 16 bytes with 16-byte aligned table and output (embedding lookups): one
// workgroup per (outer, t) row, each thread copying 16-byte chunks t, t + 256, ... of it, so a
// row of 768 floats is one load and one store per thread spread over three waves. (A wave that
// carried a whole row in a per-thread array of chunks was five times slower: the compiler kept
// the array in LDS.) Out-of-range indices set the flag and leave their row unwritten, as
// gather_kernel does.
__global__ void __launch_bounds__(256) gather_rows16_kernel(const uint4 *src, const void *idx, int idx_dtype,
                                                            long outer, long dim, long n, long inner16,
                                                            uint4 *out, int *flag) {
    for (long row = blockIdx.x; row < outer * n; row += gridDim.x) {
        const long o = row / n, t = row - o * n;
        long k = idx_dtype == MGC_I64 ? static_cast<const long long *>(idx)[t]
                                      : (long)static_cast<const int *>(idx)[t];
        if (k < 0) k += dim;
        if (k < 0 || k >= dim) {
            if (threadIdx.x == 0) *flag = 1;
            continue;
        }
        const uint4 *s = src + (o * dim + k) * inner16;
        uint4 *d = out + row * inner16;
        for (long w = threadIdx.x; w < inner16; w += 256) d[w] = s[w];
    }
}

template <typename T>
__global__ void range_kernel(const T *start, const T *delta, long n, T *out) {
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n;
         i += (long)gridDim.x * blockDim.x)
        out[i] = (T)(start[0] + (T)i * delta[0]);
}

}  // namespace mgc

using namespace mgc;

extern "C" void mgc_hip_elementwise(mgc_hip_exec *x, const mgc_hip_ew_args *args) {
    long total = 1;
    for (int d = 0; d < args->rank; ++d) total *= args->dims[d];
    if (total <= 0) return;
    mgc_hip_ew_args coalesced = *args;
    ew_coalesce(coalesced);
    const mgc_hip_ew_args *e = &coalesced;
    EwF32Args f;
    bool vec = false;
    const int nl = e->n_leaves <= 2 && e->n_instr <= 1 ? 2 : e->n_leaves <= 3 && e->n_instr <= 2 ? 3 : EWF_LEAVES;
    if (ew_f32_plan(e, f, vec, nl)) {
        const dim3 grid(blocks_for(f.units, 256, 8192));
        if (nl == 2) {
            if (vec) MGC_LAUNCH(x, (ew_f32_kernel<true, 2, 1>), grid, dim3(256), 0, f);
            else MGC_LAUNCH(x, (ew_f32_kernel<false, 2, 1>), grid, dim3(256), 0, f);
        } else if (nl == 3) {
            if (vec) MGC_LAUNCH(x, (ew_f32_kernel<true, 3, 2>), grid, dim3(256), 0, f);
            else MGC_LAUNCH(x, (ew_f32_kernel<false, 3, 2>), grid, dim3(256), 0, f);
        } else {
            if (vec) MGC_LAUNCH(x, (ew_f32_kernel<true, EWF_LEAVES, EWF_INSTR>), grid, dim3(256), 0, f);
            else MGC_LAUNCH(x, (ew_f32_kernel<false, EWF_LEAVES, EWF_INSTR>), grid, dim3(256), 0, f);
        }
        return;
    }
    MGC_LAUNCH(x, ew_program_kernel, dim3(blocks_for(total, 256, 8192)), dim3(256), 0, *e);
}

extern "C" void mgc_hip_copy(mgc_hip_exec *x, const mgc_hip_copy_args *c) {
    long total = 1;
    for (int d = 0; d < c->rank; ++d) total *= c->dims[d];
    if (total <= 0) return;
    mgc_hip_copy_args a = *c;
    TransposeGeo tg;
    dim3 tgrid;
    if (transpose_plan(a, tg, tgrid)) {
        const long per = 16 / a.elem_bytes;
        const bool vec = tg.np % per == 0 && tg.nq % per == 0 && tg.in_q % per == 0 && tg.out_p % per == 0 &&
                         tg.in_b0 % per == 0 && tg.in_b1 % per == 0 && tg.out_b0 % per == 0 &&
                         tg.out_b1 % per == 0 && tg.in_base % per == 0 && tg.out_base % per == 0 &&
                         (((uintptr_t)a.in | (uintptr_t)a.out) & 15) == 0;
        if (vec && a.elem_bytes == 4)
            MGC_LAUNCH(x, transpose_tiled_vec_kernel<unsigned>, tgrid, dim3(256), 0, tg,
                       static_cast<const unsigned *>(a.in), static_cast<unsigned *>(a.out));
        else if (vec)
            MGC_LAUNCH(x, transpose_tiled_vec_kernel<unsigned long long>, tgrid, dim3(256), 0, tg,
                       static_cast<const unsigned long long *>(a.in), static_cast<unsigned long long *>(a.out));
        else if (a.elem_bytes == 4)
            MGC_LAUNCH(x, transpose_tiled_kernel<unsigned>, tgrid, dim3(256), 0, tg,
                       static_cast<const unsigned *>(a.in), static_cast<unsigned *>(a.out));
        else
            MGC_LAUNCH(x, transpose_tiled_kernel<unsigned long long>, tgrid, dim3(256), 0, tg,
                       static_cast<const unsigned long long *>(a.in), static_cast<unsigned long long *>(a.out));
        return;
    }
    // Move 16-byte units when the innermost dim is contiguous on both sides, a multiple of the
    // unit, and every stride and base keeps the unit aligned.
    int r = a.rank;
    if (r >= 1 && a.elem_bytes <= 8 && a.in_strides[r - 1] == 1 && a.out_strides[r - 1] == 1 &&
        a.in_mod[r - 1] == 0) {
        long per = 16 / a.elem_bytes;
        bool ok = a.dims[r - 1] % per == 0 && a.in_base % per == 0 && a.out_base % per == 0 &&
                  ((uintptr_t)a.in & 15) == 0 && ((uintptr_t)a.out & 15) == 0;
        for (int d = 0; d < r - 1 && ok; ++d)
            ok = a.in_strides[d] % per == 0 && a.out_strides[d] % per == 0 &&
                 (a.in_mod[d] == 0);
        if (ok) {
            a.dims[r - 1] /= per;
            for (int d = 0; d < r - 1; ++d) {
                a.in_strides[d] /= per;
                a.out_strides[d] /= per;
            }
            a.in_base /= per;
            a.out_base /= per;
            a.elem_bytes = 16;
            total /= per;
        }
    }
    dim3 grid(blocks_for(total, 256, 8192));
    switch (a.elem_bytes) {
    case 1: MGC_LAUNCH(x, copy_kernel<unsigned char>, grid, dim3(256), 0, a); break;
    case 2: MGC_LAUNCH(x, copy_kernel<unsigned short>, grid, dim3(256), 0, a); break;
    case 4: MGC_LAUNCH(x, copy_kernel<unsigned>, grid, dim3(256), 0, a); break;
    case 8: MGC_LAUNCH(x, copy_kernel<unsigned long long>, grid, dim3(256), 0, a); break;
    default: MGC_LAUNCH(x, copy_kernel<uint4>, grid, dim3(256), 0, a); break;
    }
}

extern "C" void mgc_hip_space_to_depth(mgc_hip_exec *x, int N, int C, int H, int W, const float *in,
                                       float *out) {
    const long total = (long)N * (H / 2) * (W / 2);
    if (N <= 0 || C < 1 || C > 8 || H % 2 || W % 2 || H <= 0 || W <= 0 ||
        total * 4 * C >= 0x7fffffffL || (((uintptr_t)in & 7) | ((uintptr_t)out & 15))) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_space_to_depth: unsupported shape or alignment", hipErrorInvalidValue);
        return;
    }
    if (C <= 4 && W % 4 == 0 && ((uintptr_t)in & 15) == 0) {
        const long pairs = total / 2;
        // three 64-pair blocks per wave, so that each wave's reads overlap its previous writes
        const dim3 grid(blocks_for((pairs + 2) / 3, 256, 16384));
        const FastDiv dw4 = make_fastdiv((unsigned)(W / 4)), dh2 = make_fastdiv((unsigned)(H / 2));
        switch (C) {
        case 1: MGC_LAUNCH(x, space_to_depth_vec_kernel<1>, grid, dim3(256), 0, H / 2, W / 4, (int)pairs, dw4, dh2, in, out); break;
        case 2: MGC_LAUNCH(x, space_to_depth_vec_kernel<2>, grid, dim3(256), 0, H / 2, W / 4, (int)pairs, dw4, dh2, in, out); break;
        case 3: MGC_LAUNCH(x, space_to_depth_vec_kernel<3>, grid, dim3(256), 0, H / 2, W / 4, (int)pairs, dw4, dh2, in, out); break;
        default: MGC_LAUNCH(x, space_to_depth_vec_kernel<4>, grid, dim3(256), 0, H / 2, W / 4, (int)pairs, dw4, dh2, in, out); break;
        }
        return;
    }
    MGC_LAUNCH(x, space_to_depth_kernel, dim3(blocks_for(total, 256, 16384)), dim3(256), 0, C, H / 2,
               W / 2, (int)total, make_fastdiv((unsigned)(W / 2)), make_fastdiv((unsigned)(H / 2)), in, out);
}

extern "C" void mgc_hip_fill(mgc_hip_exec *x, void *out, long n, int elem_bytes, uint64_t bits) {
    if (n <= 0) return;
    dim3 grid(blocks_for(n, 256, 8192));
    switch (elem_bytes) {
    case 1:
        MGC_LAUNCH(x, fill_kernel<unsigned char>, grid, dim3(256), 0, (unsigned char *)out, n,
                   (unsigned char)bits);
        break;
    case 2:
        MGC_LAUNCH(x, fill_kernel<unsigned short>, grid, dim3(256), 0, (unsigned short *)out, n,
                   (unsigned short)bits);
        break;
    case 4:
        MGC_LAUNCH(x, fill_kernel<unsigned>, grid, dim3(256), 0, (unsigned *)out, n,
                   (unsigned)bits);
        break;
    default:
        MGC_LAUNCH(x, fill_kernel<unsigned long long>, grid, dim3(256), 0,
                   (unsigned long long *)out, n, (unsigned long long)bits);
        break;
    }
}

extern "C" void mgc_hip_gather(mgc_hip_exec *x, const void *src, const void *idx, int idx_dtype,
                               long outer, long dim, long n, long inner_bytes, void *out) {
    long rows = outer * n;
    if (rows <= 0 || inner_bytes <= 0) return;
    if (inner_bytes % 16 == 0 && (((uintptr_t)src | (uintptr_t)out) & 15) == 0) {
        MGC_LAUNCH(x, gather_rows16_kernel, dim3((unsigned)(rows < 65536 ? rows : 65536)), dim3(256), 0,
                   (const uint4 *)src, idx, idx_dtype, outer, dim, n, inner_bytes / 16, (uint4 *)out, x->flag);
        return;
    }
    unsigned grid = (unsigned)(rows < 65536 ? rows : 65536);
    MGC_LAUNCH(x, gather_kernel, dim3(grid), dim3(256), 0, (const unsigned char *)src, idx,
               idx_dtype, outer, dim, n, inner_bytes, (unsigned char *)out, x->flag);
}

extern "C" void mgc_hip_range(mgc_hip_exec *x, int dtype, const void *start, const void *delta,
                              long n, void *out) {
    if (n <= 0) return;
    dim3 grid(blocks_for(n, 256, 4096));
    switch (dtype) {
    case MGC_F32:
        MGC_LAUNCH(x, range_kernel<float>, grid, dim3(256), 0, (const float *)start,
                   (const float *)delta, n, (float *)out);
        break;
    case MGC_F64:
        MGC_LAUNCH(x, range_kernel<double>, grid, dim3(256), 0, (const double *)start,
                   (const double *)delta, n, (double *)out);
        break;
    case MGC_I32:
        MGC_LAUNCH(x, range_kernel<int>, grid, dim3(256), 0, (const int *)start,
                   (const int *)delta, n, (int *)out);
        break;
    default:
        MGC_LAUNCH(x, range_kernel<long long>, grid, dim3(256), 0, (const long long *)start,
                   (const long long *)delta, n, (long long *)out);
        break;
    }
}
