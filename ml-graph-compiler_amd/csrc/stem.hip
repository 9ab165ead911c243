// The ResNet stem: a 7 x 7, stride-2 convolution of the 3-channel image into 64 channels, as
// one implicit-GEMM launch that reads the image in place through element strides (an NCHW
// graph input needs no NHWC or space-to-depth copy first).
//
// The reference's C backend runs this convolution as its generic implicit-GEMM path: the
// im2col panels are packed from the NCHW image and multiplied by the packed weights
// (src/ml_graph_compiler/codegen/c.py:1099-1226 emits mgc_gemm over an MGC_OP_CONV_NCHW
// operand; runtime/mgc_kernels.c:86-133 packs it, :370-396 multiplies). Here the packing is an
// LDS window per output tile:
//  1. A workgroup of 256 threads owns TH x 16 output pixels of one image and all 64 channels.
//     The image window those pixels read (3 channels x (2 (TH - 1) + 7) rows x 38 columns; zero
//     outside the image, as the padding says) is loaded once, coalesced (neighbouring threads
//     read neighbouring columns of one row), together with the packed weights, and both go to
//     LDS.
//  2. The contraction runs over k = (c, i, j) with the tap column j padded from 7 to 8, as 84
//     steps of v_mfma_f32_32x32x2f32; step e = (c 7 + i) 4 + q takes j = 2 q in lane half 0 and
//     j = 2 q + 1 in lane half 1, so every A operand is one LDS read at an address the step
//     fixes at compile time plus the lane's own (pixel, half) offset, and every B operand one
//     read of the packed weights (two n blocks in one 8-byte read when a wave owns all 64
//     channels). The window's row pitch of 48 floats puts the 32 pixels (two rows of 16) a wave
//     reads per step in 32 different bank pairs.
//  3. The accumulators go through LDS (in the weights' space) and leave as 16-byte stores of
//     whole pixel rows, with the bias and activation applied on the way (the folded BatchNorm
//     and ReLU of the graph).
// TH = 8 (128 pixels: wave w owns tile rows 2 w, 2 w + 1 and both 32-channel blocks) for large
// batches; TH = 4 (64 pixels: wave w owns rows 2 (w / 2), 2 (w / 2) + 1 and channel block
// w % 2) spreads a small batch over twice the workgroups.
#include "mgc_device.h"

#include <stdio.h>

namespace mgc {

typedef float floatx16s __attribute__((ext_vector_type(16)));
typedef float f4s __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) f4s gf4s;

constexpr int kCsC = 3;                          // image channels
constexpr int kCsK = 7;                          // window rows and columns
constexpr int kCsS = 2;                          // stride
constexpr int kCsCout = 64;                      // output channels
constexpr int kCsSteps = kCsC * kCsK * 4;        // k pairs (c, i, q): tap columns 2 q, 2 q + 1
constexpr int kCsTW = 16;                        // output columns per tile
constexpr int kCsWC = kCsS * (kCsTW - 1) + 8;    // window columns a tile reads: 38
constexpr int kCsPitch = 48;                     // window row pitch (floats)
constexpr int kCsWFloats = kCsSteps * 128;       // packed weights: [step][32 lanes][2 halves][2 n blocks]
constexpr int kCsSP = 72;                        // staging row pitch (floats) per output pixel

struct CsDev {
    const float *img;
    unsigned sn, sc, sh, sw;  // element strides of image, channel, row and column
    int H, W, PT, PL;
    int OH, OW, tiles_h, tiles_w;
    long img_bytes;           // bytes from img to the last element the strides reach
    const float *w;           // packed weights
    const float *bias;        // [64] or null
    float *out;               // NHWC, ldc floats per pixel
    long ldc;
    int act;
    float lo, hi;
};

template <int TH>
__global__ void __launch_bounds__(256) gemm_stem_kernel(const CsDev d) {
    constexpr int WR = kCsS * (TH - 1) + kCsK;  // window rows
    constexpr int PLANE = WR * kCsPitch;
    constexpr int WIN_ELEMS = kCsC * WR * kCsWC;
    constexpr int NPIX = TH * kCsTW;
    constexpr int WQUADS = kCsWFloats / 4;
    constexpr int WQ_PER = (WQUADS + 255) / 256;
    constexpr int WIN_PER = (WIN_ELEMS + 255) / 256;
    static_assert(NPIX * kCsSP <= kCsWFloats, "the staged outputs fit the weights' space");
    __shared__ __attribute__((aligned(16))) float lds[kCsWFloats + kCsC * PLANE];
    float *const wl = lds;
    float *const win = lds + kCsWFloats;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, lh = lane >> 5;

    // neighbouring tiles of one image (whose windows overlap) run on one XCD
    const int blk = xcd_block();
    const int per_img = d.tiles_h * d.tiles_w;
    const int n = blk / per_img;
    const int rem = blk - n * per_img;
    const int ty = rem / d.tiles_w;
    const int oy0 = ty * TH, ox0 = (rem - ty * d.tiles_w) * kCsTW;
    const int iy0 = oy0 * kCsS - d.PT, ix0 = ox0 * kCsS - d.PL;

    // 1. every load of the tile goes out before the first is used: the packed weights (16-byte
    // loads) and the image window (four-byte buffer loads; an element outside the image gets an
    // offset past the resource's end and reads as zero)
    f4s wq[WQ_PER];
#pragma unroll
    for (int u = 0; u < WQ_PER; ++u) {
        const int e = tid + 256 * u;
        if (e < WQUADS) wq[u] = *(gf4s *)(d.w + 4 * e);
    }
    constexpr unsigned OOB = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rimg =
        __builtin_amdgcn_make_buffer_rsrc((void *)d.img, (short)0, (int)d.img_bytes, 0x00020000);
    const unsigned ibase = (unsigned)n * d.sn;
    float wv[WIN_PER];
#pragma unroll
    for (int u = 0; u < WIN_PER; ++u) {
        const int e = tid + 256 * u;
        const int c = e / (WR * kCsWC), r0 = e - c * (WR * kCsWC);
        const int r = r0 / kCsWC, col = r0 - r * kCsWC;
        const int y = iy0 + r, x = ix0 + col;
        const bool in = e < WIN_ELEMS && (unsigned)y < (unsigned)d.H && (unsigned)x < (unsigned)d.W;
        const unsigned off = in ? (ibase + (unsigned)c * d.sc + (unsigned)y * d.sh + (unsigned)x * d.sw) * 4u : OOB;
        wv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rimg, off, 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < WQ_PER; ++u) {
        const int e = tid + 256 * u;
        if (e < WQUADS) *reinterpret_cast<f4s *>(&wl[4 * e]) = wq[u];
    }
#pragma unroll
    for (int u = 0; u < WIN_PER; ++u) {
        const int e = tid + 256 * u;
        if (e < WIN_ELEMS) {
            const int c = e / (WR * kCsWC), r0 = e - c * (WR * kCsWC);
            const int r = r0 / kCsWC, col = r0 - r * kCsWC;
            win[c * PLANE + r * kCsPitch + col] = wv[u];
        }
    }
    __syncthreads();

    // 2. the contraction. TH = 8: wave w owns pixels 32 w .. 32 w + 31 and both n blocks;
    // TH = 4: pixels 32 (w / 2) .. + 31 and n block w % 2. Lane li is pixel (row, column)
    // (li / 16, li % 16) of the wave's two rows.
    constexpr bool BOTH = TH == 8;
    const int pb = BOTH ? wave : wave >> 1;
    const int nb = BOTH ? 0 : wave & 1;
    const float *const wa = win + (2 * pb + (li >> 4)) * kCsS * kCsPitch + kCsS * (li & 15) + lh;
    const float *const wb = wl + (li * 2 + lh) * 2 + nb;
    floatx16s acc0, acc1;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc0[r] = acc1[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < kCsC; ++c)
#pragma unroll
        for (int i = 0; i < kCsK; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = (c * kCsK + i) * 4 + q;
                const float a = wa[c * PLANE + i * kCsPitch + 2 * q];
                if constexpr (BOTH) {
                    const float2 b = *reinterpret_cast<const float2 *>(&wb[e * 128]);
                    acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b.x, acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b.y, acc1, 0, 0, 0);
                } else {
                    acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a, wb[e * 128], acc0, 0, 0, 0);
                }
            }

    // 3. register r of lane (li, lh) is pixel 8 (r / 4) + 4 lh + r % 4 of the wave's 32, channel
    // li of its n block; staged as [pixel][64] (pitch 72: lane halves 32 banks apart)
    __syncthreads();  // every wave is past its last read of the weights
    float *const stg = lds;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int pix = 32 * pb + 8 * (r >> 2) + 4 * lh + (r & 3);
        stg[pix * kCsSP + 32 * nb + li] = acc0[r];
        if constexpr (BOTH) stg[pix * kCsSP + 32 + li] = acc1[r];
    }
    __syncthreads();
    const int q4 = tid & 15;  // the channel quad this thread stores (the same for every pixel it takes)
    const f4s zero4 = {0.f, 0.f, 0.f, 0.f};
    const f4s b4 = d.bias ? *(gf4s *)(d.bias + 4 * q4) : zero4;
#pragma unroll
    for (int u = 0; u < NPIX * 16 / 256; ++u) {
        const int pix = (tid >> 4) + 16 * u;
        const int oy = oy0 + (pix >> 4), ox = ox0 + (pix & 15);
        if (oy < d.OH && ox < d.OW) {
            f4s v = *reinterpret_cast<const f4s *>(&stg[pix * kCsSP + 4 * q4]) + b4;
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = apply_act(v[t], d.act, d.lo, d.hi);
            *reinterpret_cast<f4s *>(d.out + (((long)n * d.OH + oy) * d.OW + ox) * d.ldc + 4 * q4) = v;
        }
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
    const int th = a->tile_rows == 4 || a->tile_rows == 8 ? a->tile_rows : 0;
    const int th_auto = (long)a->N * ((a->OH + 7) / 8) * ((a->OW + kCsTW - 1) / kCsTW) < 512 ? 4 : 8;
    const int TH = th ? th : th_auto;
    const long tiles = (long)a->N * ((a->OH + TH - 1) / TH) * ((a->OW + kCsTW - 1) / kCsTW);
    const bool ok = geo && st->img && ((uintptr_t)st->img & 3) == 0 && img_bytes > 0 && img_bytes < 0x7fffffffL &&
                    (a->tile_rows == 0 || th != 0) && a->w && ((uintptr_t)a->w & 15) == 0 &&
                    ((uintptr_t)a->bias & 15) == 0 && a->out && ((uintptr_t)a->out & 15) == 0 &&
                    a->ldc >= kCsCout && a->ldc % 4 == 0 && tiles < 0x7fffffffL &&
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
    d.tiles_h = (a->OH + TH - 1) / TH;
    d.tiles_w = (a->OW + kCsTW - 1) / kCsTW;
    d.img_bytes = img_bytes;
    d.w = a->w;
    d.bias = a->bias;
    d.out = a->out;
    d.ldc = a->ldc;
    d.act = a->act;
    d.lo = a->lo;
    d.hi = a->hi;
    if (TH == 8)
        MGC_LAUNCH(x, gemm_stem_kernel<8>, dim3((unsigned)tiles), dim3(256), 0, d);
    else
        MGC_LAUNCH(x, gemm_stem_kernel<4>, dim3((unsigned)tiles), dim3(256), 0, d);
}
