// Input layer of a spiking CNN and layout conversion (gfx950).
//
// snnk_conv3x3_image_lif: a static image [B][Cin][H][W] (fp32, Cin small,
// e.g. RGB) is presented at every one of T steps (the VGG16-SNN input
// convention, examples/vgg16_snn/vgg16_test.py:243 and BASELINE's config).
// The conv output is therefore the same at every step: it is computed once
// per (pixel, channel) in fp32 on the VALU (K = 9*Cin is far too small for
// MFMA) and the LIF recurrence runs T times on that constant current.
// Cout % 8 == 0 and the folded weights (9*Cin*Cout fp32) fit 64 KB of LDS.
// Output spikes go to NHWC bf16 [T][B][H][W][Cout] for the next MFMA layer,
// or (snnk_conv3x3_image_lif_act, SNNK_ACT_BITS) to packed words
// [T][B][H][W][Cout/32].
//
// snnk_to_nhwc_bf16: [N][C][HW] (fp32/bf16/f16/u8) -> [N][HW][C] bf16.
#include <type_traits>

#include "snnk_common.h"

namespace snnk {
namespace {

// One thread per run of P consecutive output pixels along x and group
// of 8 output channels, channel group fastest: the 8 lanes of a pixel run
// share its image reads (broadcast), each weight read from LDS feeds P
// FMAs, and a spike store of 8 lanes is one full 128-byte line.  The folded
// weights of all output channels sit in LDS as [cin*9 + tap][Cout], staged
// with every global read of a thread issued before its LDS writes (the
// reads follow w's [Cout][K] order, so they coalesce).  Input channels go in
// chunks of CC: a chunk's image reads (3 rows x (P+2) columns per channel)
// are all issued before its FMAs, the first chunk's while the block stages
// the weights.  Runs of P = 4 pixels (W % 4 == 0) while the grid still gives
// every SIMD 1.5 waves, runs of 2 (W % 2 == 0) while it gives one, else
// single pixels: at 32x32 images, B=32 takes 13.0 us with runs of 2 against
// 13.8 us with runs of 4 (one wave per SIMD, nothing to hide its loads
// behind), B=56 16.6 us with runs of 4 against 18.1 us with runs of 2.
constexpr int kImgG = 8;
constexpr int kImgMaxLds = 64 * 1024;

// v of the lane CTRL names within each group of 4 lanes (DPP quad_perm)
template <int CTRL>
__device__ __forceinline__ uint32_t quad_lane(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// BITS: spikes as packed words [T][B][H][W][Cout/32] (bit c%32 of word c/32):
// the 4 lanes of a quad hold channel groups 4w..4w+3 of one pixel run
// (Cout % 32 == 0 makes the groups per run a multiple of 4), so their 8-bit
// spike sets OR into word w over two DPP exchanges.
template <int P, int CC, bool BITS>
__global__ __launch_bounds__(256) void conv_image_lif_kernel(
    const float* __restrict__ img, const float* __restrict__ w, const float* __restrict__ bias,
    uint16_t* __restrict__ out, int T, int n_pix, int Cin, int H, int W, int Cout, float decay,
    float in_scale, float vth, float v_reset, int soft_reset) {
  extern __shared__ float wl[];
  const int K = Cin * 9;
  const int groups = Cout / kImgG;
  const int n_runs = n_pix / P;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const bool live = gid < static_cast<int64_t>(n_runs) * groups;
  const int g0 = live ? static_cast<int>(gid) : 0;  // threads past the end stage weights only
  const int run = g0 / groups;
  const int p = run * P;  // first pixel (b, y, x) of the run
  const int n0 = (g0 - run * groups) * kImgG;
  const int HW = H * W;
  const int b = p / HW;
  const int r = p - b * HW;
  const int y = r / W, x = r - y * W;

  // image taps of one channel chunk: rows y-1..y+1, columns x-1..x+P
  // (zero outside the image or past Cin).  Every read goes to the tap's
  // position clamped into the image (and channel 0 past Cin), so it is in
  // bounds and needs no branch; the select then zeroes the taps outside.
  float xin[CC][3][P + 2];
  auto load_chunk = [&](int c0) {
#pragma unroll
    for (int cc = 0; cc < CC; ++cc) {
      const int c = c0 + cc;
      const float* ip = img + (static_cast<int64_t>(b) * Cin + (c < Cin ? c : 0)) * HW;
#pragma unroll
      for (int dy = 0; dy < 3; ++dy) {
        const int ys = y + dy - 1;
        const int yc = ys < 0 ? 0 : ys >= H ? H - 1 : ys;
#pragma unroll
        for (int dx = 0; dx < P + 2; ++dx) {
          const int xs = x + dx - 1;
          const int xc = xs < 0 ? 0 : xs >= W ? W - 1 : xs;
          const bool in = live && c < Cin && ys >= 0 && ys < H && xs >= 0 && xs < W;
          const float v = ip[yc * W + xc];
          xin[cc][dy][dx] = in ? v : 0.0f;
        }
      }
    }
  };
  load_chunk(0);
  constexpr int kStageU = 8;
  for (int i0 = 0; i0 < K * Cout; i0 += 256 * kStageU) {
    float tmp[kStageU];
#pragma unroll
    for (int u = 0; u < kStageU; ++u) {
      const int i = i0 + u * 256 + threadIdx.x;
      tmp[u] = i < K * Cout ? w[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kStageU; ++u) {
      const int i = i0 + u * 256 + threadIdx.x;
      if (i < K * Cout) {
        const int n = i / K, k = i - n * K;
        wl[k * Cout + n] = tmp[u];
      }
    }
  }
  __syncthreads();
  if (!live) return;

  float acc[P][kImgG];
#pragma unroll
  for (int q = 0; q < P; ++q)
#pragma unroll
    for (int j = 0; j < kImgG; ++j) acc[q][j] = 0.0f;
  for (int c0 = 0; c0 < Cin; c0 += CC) {
    if (c0 > 0) load_chunk(c0);
#pragma unroll
    for (int cc = 0; cc < CC; ++cc) {
      if (c0 + cc >= Cin) break;
#pragma unroll
      for (int tap = 0; tap < 9; ++tap) {
        const float* wk = wl + ((c0 + cc) * 9 + tap) * Cout + n0;
        float wv[kImgG];
#pragma unroll
        for (int j = 0; j < kImgG; ++j) wv[j] = wk[j];
#pragma unroll
        for (int q = 0; q < P; ++q)
#pragma unroll
          for (int j = 0; j < kImgG; ++j)
            acc[q][j] = __builtin_fmaf(xin[cc][tap / 3][tap % 3 + q], wv[j], acc[q][j]);
      }
    }
  }
  float bv[kImgG];
#pragma unroll
  for (int j = 0; j < kImgG; ++j) bv[j] = bias ? bias[n0 + j] : 0.0f;

  const int64_t step = static_cast<int64_t>(n_pix) * Cout;
#pragma unroll
  for (int q = 0; q < P; ++q) {
    float u[kImgG], v[kImgG];
#pragma unroll
    for (int j = 0; j < kImgG; ++j) {
      u[j] = bias ? acc[q][j] + bv[j] : acc[q][j];
      v[j] = 0.0f;
    }
    uint16_t* o = out + static_cast<int64_t>(p + q) * Cout + n0;
    uint32_t* ow = reinterpret_cast<uint32_t*>(out) + static_cast<int64_t>(p + q) * (Cout / 32) +
                   n0 / 32;
    for (int t = 0; t < T; ++t) {
      uint32_t bits[kImgG / 2];
      uint32_t byte = 0;
#pragma unroll
      for (int j = 0; j < kImgG; ++j) {
        const float h = __fadd_rn(__fmul_rn(decay, v[j]), __fmul_rn(in_scale, u[j]));
        const bool s = h >= vth;
        v[j] = s ? (soft_reset ? __fsub_rn(h, vth) : v_reset) : h;
        const uint32_t sb = s ? 0x3F80u : 0u;
        if (j & 1) bits[j / 2] |= sb << 16;
        else bits[j / 2] = sb;
        byte |= s ? 1u << j : 0u;
      }
      if constexpr (BITS) {
        uint32_t wd = byte << (8 * ((n0 / kImgG) & 3));
        wd |= quad_lane<0xB1>(wd);  // lane ^ 1
        wd |= quad_lane<0x4E>(wd);  // lane ^ 2
        if (((n0 / kImgG) & 3) == 0) ow[t * (step / 32)] = wd;
      } else {
        *reinterpret_cast<u32x4*>(o + t * step) = u32x4{bits[0], bits[1], bits[2], bits[3]};
      }
    }
  }
}

template <typename Raw>
__device__ __forceinline__ uint16_t to_bf16_bits(Raw v);
template <> __device__ __forceinline__ uint16_t to_bf16_bits<float>(float v) {
  // round to nearest even (inputs here are finite)
  uint32_t u = __float_as_uint(v);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
template <> __device__ __forceinline__ uint16_t to_bf16_bits<uint8_t>(uint8_t v) {
  return v ? 0x3F80u : 0u;
}

// 32x32 tile transpose through LDS: reads along HW, writes along C.
template <typename Raw, int KIND>  // KIND: 0 generic (float/u8), 1 bf16 copy, 2 f16
__global__ __launch_bounds__(256) void to_nhwc_kernel(const Raw* __restrict__ src,
                                                      uint16_t* __restrict__ dst, int64_t C,
                                                      int64_t HW) {
  __shared__ uint16_t tile[32][33];
  const int64_t n = blockIdx.z;
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int i = ty; i < 32; i += 8) {
    const int64_t c = c0 + i, p = p0 + tx;
    uint16_t v = 0;
    if (c < C && p < HW) {
      const Raw r = src[(n * C + c) * HW + p];
      if constexpr (KIND == 0) v = to_bf16_bits<Raw>(r);
      else if constexpr (KIND == 1) v = r;
      else v = to_bf16_bits<float>(static_cast<float>(__builtin_bit_cast(_Float16, r)));
    }
    tile[i][tx] = v;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int64_t p = p0 + i, c = c0 + tx;
    if (c < C && p < HW) dst[(n * HW + p) * C + c] = tile[tx][i];
  }
}

}  // namespace
}  // namespace snnk

using namespace snnk;

extern "C" int snnk_conv3x3_image_lif_act(const float* image, const float* w, const float* bias,
                                          void* spikes_out, int32_t out_fmt, int64_t T,
                                          int64_t B, int64_t Cin, int64_t H, int64_t W,
                                          int64_t Cout, float decay, float in_scale,
                                          float v_threshold, float v_reset, int32_t soft_reset,
                                          void* stream) {
  if (T < 0 || B < 0 || Cin <= 0 || H < 0 || W < 0 || Cout <= 0) return SNNK_EINVAL;
  if (out_fmt != SNNK_ACT_BF16 && out_fmt != SNNK_ACT_BITS) return SNNK_EINVAL;
  if (T == 0 || B == 0 || H == 0 || W == 0) return SNNK_OK;
  if (image == nullptr || w == nullptr || spikes_out == nullptr) return SNNK_EINVAL;
  const bool bits = out_fmt == SNNK_ACT_BITS;
  // channel groups of 8 are stored as 16-byte vectors (packed: 32-channel
  // words); all folded weights must fit the kernel's LDS
  const int64_t lds = Cin * 9 * Cout * 4;
  if (Cout % (bits ? 32 : kImgG) != 0 || lds > kImgMaxLds) return SNNK_EUNSUPPORTED;
  if (B * H * W > 0x7FFFFFFFll || B * H * W * Cin > (1ll << 40) ||
      T * B * H * W * Cout > (1ll << 40))
    return SNNK_EUNSUPPORTED;
  if (!aligned(spikes_out, 16)) return SNNK_EALIGN;
  const int64_t n_pix = B * H * W;
  // pixels per thread (see the kernel's comment); 256 * 256 threads are one
  // wave per SIMD of the 256 CUs
  const int64_t units = n_pix * (Cout / kImgG);
  const int run = (W % 4 == 0 && units / 4 >= 3 * 256 * 128) ? 4
                  : (W % 2 == 0 && units / 2 >= 256 * 256)   ? 2
                                                               : 1;
  const int64_t blocks = (n_pix / run * (Cout / kImgG) + 255) / 256;
  if (blocks > 0x7FFFFFFFll) return SNNK_EUNSUPPORTED;
  // channel chunk: 3 for RGB-like inputs, else 4
  const bool c3 = Cin % 3 == 0;
  auto pick = [&](auto bits_tag) {
    constexpr bool kBits = decltype(bits_tag)::value;
    return run == 4   ? (c3 ? conv_image_lif_kernel<4, 3, kBits> : conv_image_lif_kernel<4, 4, kBits>)
           : run == 2 ? (c3 ? conv_image_lif_kernel<2, 3, kBits> : conv_image_lif_kernel<2, 4, kBits>)
                      : (c3 ? conv_image_lif_kernel<1, 3, kBits> : conv_image_lif_kernel<1, 4, kBits>);
  };
  auto kern = bits ? pick(std::true_type{}) : pick(std::false_type{});
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(256),
                     static_cast<unsigned>(lds), static_cast<hipStream_t>(stream), image, w,
                     bias, static_cast<uint16_t*>(spikes_out), static_cast<int>(T),
                     static_cast<int>(n_pix), static_cast<int>(Cin), static_cast<int>(H),
                     static_cast<int>(W), static_cast<int>(Cout), decay, in_scale, v_threshold,
                     v_reset, soft_reset ? 1 : 0);
  return launch_status();
}

extern "C" int snnk_conv3x3_image_lif(const float* image, const float* w, const float* bias,
                                      uint16_t* spikes_out, int64_t T, int64_t B, int64_t Cin,
                                      int64_t H, int64_t W, int64_t Cout, float decay,
                                      float in_scale, float v_threshold, float v_reset,
                                      int32_t soft_reset, void* stream) {
  return snnk_conv3x3_image_lif_act(image, w, bias, spikes_out, SNNK_ACT_BF16, T, B, Cin, H, W,
                                    Cout, decay, in_scale, v_threshold, v_reset, soft_reset,
                                    stream);
}

extern "C" int snnk_to_nhwc_bf16(const void* src, int32_t src_dtype, uint16_t* dst, int64_t N,
                                 int64_t C, int64_t HW, void* stream) {
  if (N < 0 || C < 0 || HW < 0) return SNNK_EINVAL;
  if (N == 0 || C == 0 || HW == 0) return SNNK_OK;
  if (src == nullptr || dst == nullptr) return SNNK_EINVAL;
  const int64_t gx = (HW + 31) / 32, gy = (C + 31) / 32;
  if (gx > 0x7FFFFFFFll || gy > 65535 || N > 65535) return SNNK_EUNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(gx, gy, N);
  switch (src_dtype) {
    case SNNK_F32:
      hipLaunchKernelGGL((to_nhwc_kernel<float, 0>), grid, dim3(256), 0, s,
                         static_cast<const float*>(src), dst, C, HW);
      break;
    case SNNK_U8:
      hipLaunchKernelGGL((to_nhwc_kernel<uint8_t, 0>), grid, dim3(256), 0, s,
                         static_cast<const uint8_t*>(src), dst, C, HW);
      break;
    case SNNK_BF16:
      hipLaunchKernelGGL((to_nhwc_kernel<uint16_t, 1>), grid, dim3(256), 0, s,
                         static_cast<const uint16_t*>(src), dst, C, HW);
      break;
    case SNNK_F16:
      hipLaunchKernelGGL((to_nhwc_kernel<uint16_t, 2>), grid, dim3(256), 0, s,
                         static_cast<const uint16_t*>(src), dst, C, HW);
      break;
    default:
      return SNNK_EINVAL;
  }
  return launch_status();
}
