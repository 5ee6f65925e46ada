// Classifier head averaged over time, on packed spike words (gfx950).
//
// snnk_linear_mean_t_bits: out[r][n] = (1/T) sum_t (x[t][r] . w[n]) + bias[n]
// for a head with few outputs (N <= 64), x packed spike words [T][R][K/32]
// (bit k%32 of word k/32).  The spikes are 0/1, so sum_t x[t][r][k] is a
// spike count c[k] in 0..T and the head is one dot product per (r, n),
// sum_k c[k] * w[n][k], instead of T of them: the K loop runs once, on the
// VALU (N is far below an MFMA tile), in one block per row.
//
// Thread j takes inputs 16h .. 16h+15 for h = j, j + 256, ...: it counts each
// input's spikes over the T steps from the T half-words, then adds count *
// weight into its sums (NMAX of them, a multiple of 8, at least N).  The 256
// partial sums of each output are reduced in a fixed order (lanes by xor
// shuffles, then the four waves in order), so repeated calls give identical
// results.
#include "snnk_common.h"

namespace snnk {
namespace {

constexpr int kHeadThreads = 256;
constexpr int kHeadMaxN = 64;

template <int NMAX>
__global__ __launch_bounds__(kHeadThreads) void head_mean_bits_kernel(
    const uint32_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ out, int T, int R, int K, int N) {
  __shared__ float part[kHeadThreads / 64][NMAX];
  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int KW = K >> 5;
  float acc[NMAX];
#pragma unroll
  for (int n = 0; n < NMAX; ++n) acc[n] = 0.0f;

  for (int h = tid; h < 2 * KW; h += kHeadThreads) {
    const int j = h >> 1, sh = (h & 1) * 16;
    // 16 bf16 weights per output, two 16-byte loads (K % 32 == 0 keeps them
    // aligned); rows in batches of 8, a batch's loads issued before its
    // products (rows past N repeat row N - 1; their sums are never read).
    // The first two batches are loaded before the spike words are counted,
    // so that the memory round trips overlap; later batches reuse the two
    // register slots.
    const uint16_t* wk = w + 16 * h;
    u32x4 wv[2][8][2];
    auto load_w = [&](int slot, int n0) __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t row = n0 + e < N ? n0 + e : N - 1;
        wv[slot][e][0] = *reinterpret_cast<const u32x4*>(wk + row * K);
        wv[slot][e][1] = *reinterpret_cast<const u32x4*>(wk + row * K + 8);
      }
    };
    load_w(0, 0);
    if (N > 8) load_w(1, 8);
    // spike count of each of the 16 inputs over the T steps; the words of
    // four steps are loaded (from step T - 1 for steps past the last, then
    // zeroed: no branch, no wait between the loads) before they are counted
    float c[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) c[b] = 0.0f;
    for (int t0 = 0; t0 < T; t0 += 4) {
      uint32_t wd[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = t0 + u < T ? t0 + u : T - 1;
        wd[u] = x[(static_cast<int64_t>(t) * R + r) * KW + j] >> sh;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) wd[u] = t0 + u < T ? wd[u] : 0u;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int b = 0; b < 16; ++b) c[b] += static_cast<float>((wd[u] >> b) & 1u);
    }
#pragma unroll
    for (int n0 = 0; n0 < NMAX; n0 += 8) {
      if (n0 >= N) break;
      const int slot = (n0 >> 3) & 1;
      if (n0 >= 16) load_w(slot, n0);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float s = acc[n0 + e];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          s = __builtin_fmaf(c[2 * q], __uint_as_float(wv[slot][e][0][q] << 16), s);
          s = __builtin_fmaf(c[2 * q + 1], __uint_as_float(wv[slot][e][0][q] & 0xFFFF0000u), s);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          s = __builtin_fmaf(c[8 + 2 * q], __uint_as_float(wv[slot][e][1][q] << 16), s);
          s = __builtin_fmaf(c[9 + 2 * q], __uint_as_float(wv[slot][e][1][q] & 0xFFFF0000u), s);
        }
        acc[n0 + e] = s;
      }
    }
  }
  // lanes of a wave, then the waves in order
#pragma unroll
  for (int n = 0; n < NMAX; ++n) {
    if (n >= N) break;
    float v = acc[n];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    if (lane == 0) part[wave][n] = v;
  }
  __syncthreads();
  if (tid < N) {
    float v = part[0][tid];
#pragma unroll
    for (int wv = 1; wv < kHeadThreads / 64; ++wv) v += part[wv][tid];
    out[static_cast<int64_t>(r) * N + tid] =
        __fadd_rn(__fdiv_rn(v, static_cast<float>(T)), bias ? bias[tid] : 0.0f);
  }
}

}  // namespace
}  // namespace snnk

using namespace snnk;

extern "C" int snnk_linear_mean_t_bits(const uint32_t* x, const uint16_t* w, const float* bias,
                                       float* out, int64_t T, int64_t R, int64_t K, int64_t N,
                                       void* stream) {
  if (T < 0 || R < 0 || K < 0 || N < 0) return SNNK_EINVAL;
  if (R == 0 || N == 0) return SNNK_OK;
  if (out == nullptr || w == nullptr || (K > 0 && T > 0 && x == nullptr)) return SNNK_EINVAL;
  if (K % 32 != 0 || N > kHeadMaxN) return SNNK_EUNSUPPORTED;
  if (!aligned(w, 16)) return SNNK_EALIGN;
  if (T == 0) return SNNK_EINVAL;  // the mean over no steps is undefined
  if (R > 0x7FFFFFFFll || K > 0x7FFFFFFFll || T * R * (K / 32) > (1ll << 40)) return SNNK_EUNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(R)), block(kHeadThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (N <= 16)
    hipLaunchKernelGGL((head_mean_bits_kernel<16>), grid, block, 0, s, x, w, bias, out,
                       static_cast<int>(T), static_cast<int>(R), static_cast<int>(K), static_cast<int>(N));
  else if (N <= 32)
    hipLaunchKernelGGL((head_mean_bits_kernel<32>), grid, block, 0, s, x, w, bias, out,
                       static_cast<int>(T), static_cast<int>(R), static_cast<int>(K), static_cast<int>(N));
  else
    hipLaunchKernelGGL((head_mean_bits_kernel<64>), grid, block, 0, s, x, w, bias, out,
                       static_cast<int>(T), static_cast<int>(R), static_cast<int>(K), static_cast<int>(N));
  return launch_status();
}
