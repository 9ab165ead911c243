// The ResNet stem: a 7 x 7, stride-2 convolution of the 3-channel image into 64 channels, as
// one implicit-GEMM launch that reads the image in place through element strides (an NCHW
// graph input needs no NHWC or space-to-depth copy first).
//
// The reference's C backend runs this convolution as its generic implicit-GEMM path: the
// im2col panels are packed from the NCHW image and multiplied by the packed weights
// (src/ml_graph_compiler/codegen/c.py:1099-1226 emits mgc_gemm over an MGC_OP_CONV_NCHW
// operand; runtime/mgc_kernels.c:86-133 packs it, :370-396 multiplies). Here the packing is an
// LDS window per output tile:
//  * An output tile is 8 x 16 pixels of one image times all 64 channels, and a workgroup is
//    eight waves: wave w owns tile rows 2 (w / 2) and 2 (w / 2) + 1 (32 pixels, lane li =
//    pixel (li / 16, li % 16)) and channel block w % 2 (32 channels).
//  * The contraction runs over k = (c, i, j) with the tap column j padded from 7 to 8, as 84
//    steps of v_mfma_f32_32x32x2f32; step e = (c 7 + i) 4 + q takes j = 2 q in lane half 0 and
//    j = 2 q + 1 in lane half 1. Each A operand is one LDS read of the tile's image window at an
//    address the step fixes at compile time plus the lane's own (pixel, half) offset, and each B
//    operand one read of the packed weights, which sit in LDS for the whole launch. The window
//    (3 channels x 21 rows x 38 columns, zero outside the image as the padding says) has a row
//    pitch of 48 floats, which puts the 64 lanes of a read in 64 different banks.
//  * Workgroups are persistent (two per CU: 67 KB of LDS each, four waves per SIMD): each takes
//    tiles g, g + G, ... (G workgroups; neighbouring workgroups, which run on one XCD, take
//    neighbouring tiles of one image, whose windows overlap), and requests the next tile's
//    window (coalesced four-byte loads: neighbouring lanes read neighbouring columns of one
//    row) before multiplying the current one, so the load latency hides behind the MFMAs; two
//    LDS window buffers alternate.
//  * The accumulators leave straight from registers with the bias and activation applied (the
//    folded BatchNorm and ReLU of the graph): for each register, lanes 0-31 write 32
//    consecutive channels (128 bytes) of one pixel and lanes 32-63 those of another.
// Measured against the space-to-depth copy and GEMM it replaces, in the ResNet-50 forward on
// one MI355X: batch 32 2.768 -> 2.757 ms, batch 1 0.3873 -> 0.3840 ms. (A form with four waves
// per workgroup and each wave's B operand in registers, 3 waves per SIMD, measured 2.765 and
// 0.3859 ms.)
#include "mgc_device.h"

namespace mgc {

typedef float floatx16s __attribute__((ext_vector_type(16)));

constexpr int kCsC = 3;                          // image channels
constexpr int kCsK = 7;                          // window rows and columns
constexpr int kCsS = 2;                          // stride
constexpr int kCsCout = 64;                      // output channels
constexpr int kCsSteps = kCsC * kCsK * 4;        // k pairs (c, i, q): tap columns 2 q, 2 q + 1
constexpr int kCsTH = 8;                         // output rows per tile
constexpr int kCsTW = 16;                        // output columns per tile
constexpr int kCsWR = kCsS * (kCsTH - 1) + kCsK; // window rows: 21
constexpr int kCsWC = kCsS * (kCsTW - 1) + 8;    // window columns: 38
constexpr int kCsPitch = 48;                     // window row pitch (floats)
constexpr int kCsPlane = kCsWR * kCsPitch;       // one channel's window rows
constexpr int kCsWin = kCsC * kCsPlane;          // one window buffer (floats)
constexpr int kCsWFloats = kCsSteps * 128;       // packed weights: [step][32 lanes][2 halves][2 n blocks]
constexpr int kCsCUs = 256;                      // MI355X compute units
constexpr int kCsPerCU = 2;                      // workgroups a CU holds at once (67 KB of LDS each)

struct CsDev {
    const float *img;
    unsigned sn, sc, sh, sw;  // element strides of image, channel, row and column
    int H, W, PT, PL;
    int OH, OW, tiles_h, tiles_w, tiles;
    long img_bytes;           // bytes from img to the last element the strides reach
    const float *w;           // packed weights
    const float *bias;        // [64] or null
    float *out;               // NHWC, ldc floats per pixel
    long ldc;
    int act;
    float lo, hi;
};

__global__ void __launch_bounds__(512) gemm_stem_kernel(const CsDev d) {
    __shared__ __attribute__((aligned(16))) float win[2][kCsWin];
    __shared__ __attribute__((aligned(16))) float wl[kCsWFloats];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, lh = lane >> 5;
    const int pb = wave >> 1, nb = wave & 1;

    // the packed weights into LDS once per workgroup; lane (li, lh) of channel block nb reads
    // W[32 nb + li][k = 2 e + lh] of step e at wb[128 e]
    for (int e = tid; e < kCsWFloats / 4; e += 512)
        *reinterpret_cast<float4 *>(&wl[4 * e]) = *reinterpret_cast<const float4 *>(d.w + 4 * e);
    const float *const wb = wl + (li * 2 + lh) * 2 + nb;
    const float bias = d.bias ? d.bias[32 * nb + li] : 0.0f;

    constexpr unsigned OOB = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rimg =
        __builtin_amdgcn_make_buffer_rsrc((void *)d.img, (short)0, (int)d.img_bytes, 0x00020000);
    const int per_img = d.tiles_h * d.tiles_w;
    // image, first output row and column of tile t
    auto origin = [&](int t, int &n, int &oy0, int &ox0) __attribute__((always_inline)) {
        n = t / per_img;
        const int rem = t - n * per_img;
        const int ty = rem / d.tiles_w;
        oy0 = ty * kCsTH;
        ox0 = (rem - ty * d.tiles_w) * kCsTW;
    };
    // The window of tile t into registers: wave w moves window rows w, w + 8, ... (row R =
    // channel R / 21, image row R % 21 of the window), lane l column l < 38, so the row
    // arithmetic is scalar and the column bounds are tested once per tile. An element outside
    // the image gets an offset past the resource's end and reads as zero.
    constexpr int WROWS = kCsC * kCsWR;              // 63 window rows over the channels
    constexpr int RPW = (WROWS + 7) / 8;             // rows per wave
    static_assert(kCsWC <= 64, "a window row fits a wave");
    const bool col_ok = lane < kCsWC;
    auto fetch_window = [&](int t, float (&v)[RPW]) __attribute__((always_inline)) {
        int n, oy0, ox0;
        origin(t, n, oy0, ox0);
        const int iy0 = oy0 * kCsS - d.PT, ix0 = ox0 * kCsS - d.PL;
        const int x = ix0 + lane;
        const bool x_ok = col_ok && (unsigned)x < (unsigned)d.W;
        const unsigned xoff = (unsigned)n * d.sn + (unsigned)x * d.sw;
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            const int R = wave + 8 * j;
            const int c = R / kCsWR, y = iy0 + (R - c * kCsWR);
            const bool in = R < WROWS && x_ok && (unsigned)y < (unsigned)d.H;
            const unsigned off = in ? (xoff + (unsigned)c * d.sc + (unsigned)y * d.sh) * 4u : OOB;
            v[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rimg, off, 0, 0));
        }
    };
    auto place_window = [&](const float (&v)[RPW], float *buf) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            const int R = wave + 8 * j;
            const int c = R / kCsWR;
            if (R < WROWS && col_ok) buf[c * kCsPlane + (R - c * kCsWR) * kCsPitch + lane] = v[j];
        }
    };

    // neighbouring workgroups (one XCD) take neighbouring tiles
    const int G = gridDim.x;
    int t = xcd_block();
    float pv[RPW];
    if (t < d.tiles) {
        fetch_window(t, pv);
        place_window(pv, win[0]);
    }
    __syncthreads();
    const int aoff = (2 * pb + (li >> 4)) * kCsS * kCsPitch + kCsS * (li & 15) + lh;
    int cur = 0;
    for (; t < d.tiles; t += G) {
        const int tn = t + G;
        if (tn < d.tiles) fetch_window(tn, pv);

        // the contraction over the current window: A and B operands move from LDS to registers
        // a chunk of CH steps ahead of the multiplies that use them; the scheduling barriers
        // keep the compiler from sinking the reads back to their uses
        const float *const wa = win[cur] + aoff;
        floatx16s acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        constexpr int CH = 6;
        static_assert(kCsSteps % CH == 0, "whole chunks");
        float ra[2][CH], rb[2][CH];
        auto fetch_a = [&](const int ch, const int buf) __attribute__((always_inline)) {
#pragma unroll
            for (int s = 0; s < CH; ++s) {
                const int e = ch * CH + s;
                const int c = e / (kCsK * 4), i = (e / 4) % kCsK, q = e % 4;
                ra[buf][s] = wa[c * kCsPlane + i * kCsPitch + 2 * q];
                rb[buf][s] = wb[e * 128];
            }
        };
        fetch_a(0, 0);
#pragma unroll
        for (int ch = 0; ch < kCsSteps / CH; ++ch) {
            if (ch + 1 < kCsSteps / CH) fetch_a(ch + 1, (ch + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < CH; ++s)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ra[ch & 1][s], rb[ch & 1][s], acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }

        // the next window goes to the other buffer (its last readers finished before the
        // previous iteration's barrier)
        if (tn < d.tiles) place_window(pv, win[cur ^ 1]);

        // register r of lane (li, lh): pixel 8 (r / 4) + 4 lh + r % 4 of the wave's 32, channel
        // 32 nb + li; a tile wholly inside the output takes no bounds tests
        int n, oy0, ox0;
        origin(t, n, oy0, ox0);
        float *const obase = d.out + (((long)n * d.OH + oy0) * d.OW + ox0) * d.ldc + 32 * nb + li;
        const bool whole = oy0 + kCsTH <= d.OH && ox0 + kCsTW <= d.OW;
        const long row_st = (long)d.OW * d.ldc;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int pix = 32 * pb + 8 * (r >> 2) + 4 * lh + (r & 3);
            const int py = pix >> 4, px = pix & 15;
            float v = acc[r] + bias;
            v = d.act == MGC_ACT_RELU ? (v > 0.0f ? v : 0.0f) : apply_act(v, d.act, d.lo, d.hi);
            if (whole || (oy0 + py < d.OH && ox0 + px < d.OW)) obase[py * row_st + px * d.ldc] = v;
        }
        __syncthreads();
        cur ^= 1;
    }
}

}  // namespace mgc

using namespace mgc;

extern "C" int mgc_hip_conv_stem_supported(int C, int KH, int KW, int SH, int SW, int Cout) {
    return C == kCsC && KH == kCsK && KW == kCsK && SH == kCsS && SW == kCsS && Cout == kCsCout;
}

extern "C" long mgc_hip_conv_stem_weight_floats(void) { return kCsWFloats; }

extern "C" void mgc_hip_conv_stem(mgc_hip_exec *x, const mgc_hip_stem_args *st, const mgc_hip_conv_stem_args *a) {
    if (!st || !a) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_conv_stem: no arguments", hipErrorInvalidValue);
        return;
    }
    if (a->N <= 0 || a->OH <= 0 || a->OW <= 0) return;
    const bool geo = mgc_hip_conv_stem_supported(st->C, st->KH, st->KW, st->SH, st->SW, kCsCout) && st->H > 0 &&
                     st->W > 0 && st->PT >= 0 && st->PL >= 0 && st->sn >= 0 && st->sc >= 0 && st->sh >= 0 &&
                     st->sw >= 0;
    const long img_bytes = geo ? ((long)(a->N - 1) * st->sn + (long)(st->C - 1) * st->sc +
                                  (long)(st->H - 1) * st->sh + (long)(st->W - 1) * st->sw + 1) * 4
                               : -1;
    const long tiles = (long)a->N * ((a->OH + kCsTH - 1) / kCsTH) * ((a->OW + kCsTW - 1) / kCsTW);
    const bool ok = geo && st->img && ((uintptr_t)st->img & 3) == 0 && img_bytes > 0 && img_bytes < 0x7fffffffL &&
                    a->workgroups >= 0 && a->w && ((uintptr_t)a->w & 15) == 0 && a->out &&
                    ((uintptr_t)a->out & 3) == 0 && a->ldc >= kCsCout && tiles < 0x7fffffffL &&
                    (long)(st->H + kCsK) * (st->W + kCsK) < 0x40000000L;
    if (!ok) {
        x->launch_error = (int)hipErrorInvalidValue;
        set_error("mgc_hip_conv_stem: shape, layout or alignment outside its limits", hipErrorInvalidValue);
        return;
    }
    CsDev d;
    d.img = st->img;
    d.sn = (unsigned)st->sn;
    d.sc = (unsigned)st->sc;
    d.sh = (unsigned)st->sh;
    d.sw = (unsigned)st->sw;
    d.H = st->H;
    d.W = st->W;
    d.PT = st->PT;
    d.PL = st->PL;
    d.OH = a->OH;
    d.OW = a->OW;
    d.tiles_h = (a->OH + kCsTH - 1) / kCsTH;
    d.tiles_w = (a->OW + kCsTW - 1) / kCsTW;
    d.tiles = (int)tiles;
    d.img_bytes = img_bytes;
    d.w = a->w;
    d.bias = a->bias;
    d.out = a->out;
    d.ldc = a->ldc;
    d.act = a->act;
    d.lo = a->lo;
    d.hi = a->hi;
    // one round of workgroups over the CUs (two per CU), or one per tile when tiles are fewer
    const long cap = a->workgroups > 0 ? a->workgroups : (long)kCsPerCU * kCsCUs;
    const unsigned grid = (unsigned)(tiles < cap ? tiles : cap);
    MGC_LAUNCH(x, gemm_stem_kernel, dim3(grid), dim3(512), 0, d);
}
