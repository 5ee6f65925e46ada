// Spike self-attention core for gfx950: integer QK^T and (QK^T)V on int8
// MFMA (v_mfma_i32_32x32x32_i8) over {0,1} spikes, no softmax, then a
// multi-step LIF on the scaled counts.
//
// Reference: the SSA block (snn_compiler/nn/attention.py:133-164) computes
// kv = K^T V and a = (q @ kv) * scale, then attn_lif
// (spike_av_lif, snn_compiler/kernels/attention.py:49-137).  Over integers
// (Q K^T) V == Q (K^T V), so the counts are identical; this kernel uses the
// (Q K^T) V order and can return both count tensors for bit-exact checks.
//
// One block (one wave) per (batch, head).  Per step t the wave stages Q_t,
// K_t and V_t^T of its head in LDS as int8 (zero padded to 64 tokens x 64
// dims), computes S = Q K^T into accumulators, writes S to LDS as int8
// (0 <= S <= d <= 64), computes O = S V, and runs the LIF
// v = decay*v + in_scale*O on O in registers; the membrane of every
// (token, dim) stays in the same lane for all T steps.
#include "snnk_common.h"

namespace snnk {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kMaxTok = 64;
constexpr int kMaxDim = 64;
constexpr int kPitch = 80;  // LDS row pitch in bytes (conflict-free 16-byte reads)

struct AttnArgs {
  const uint16_t* q;  // bf16 spikes, element (t, b*N + n, col0 + h*d + dd)
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_row, k_row, v_row;  // row strides (elements)
  int64_t q_t, k_t, v_t;        // step strides (elements)
  uint16_t* out;                // bf16 spikes (t, b*N + n, h*d + dd)
  int64_t o_row, o_t;
  int32_t* s_counts;            // optional [T][B][H][N][N]
  int32_t* o_counts;            // optional [T][B][H][N][d]
  int T, B, H, N, d;
  float decay, in_scale, vth, v_reset;
  int soft_reset;
};

__device__ __forceinline__ int8_t bit_of(uint16_t x) { return (x & 0x7FFFu) ? 1 : 0; }

template <int NT, int DT>  // token tiles, dim tiles (32 each)
__global__ __launch_bounds__(64) void ssa_attention_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t qs[kMaxTok * kPitch];
  __shared__ __attribute__((aligned(16))) int8_t ks[kMaxTok * kPitch];
  __shared__ __attribute__((aligned(16))) int8_t vt[kMaxDim * kPitch];  // [dim][token]
  __shared__ __attribute__((aligned(16))) int8_t ss[kMaxTok * kPitch];  // S as int8

  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - b * a.H;
  const int r32 = lane & 31, g = lane >> 5;

  float vm[NT][DT][16];
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int j = 0; j < DT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) vm[i][j][e] = 0.0f;

  for (int t = 0; t < a.T; ++t) {
    // ---- stage Q_t, K_t (row = token) and V_t^T (row = dim) as int8 -------
    {
      const int n = lane;  // one token per lane
      const bool ok = n < a.N;
      const int64_t rq = static_cast<int64_t>(t) * a.q_t + (static_cast<int64_t>(b) * a.N + n) * a.q_row + h * a.d;
      const int64_t rk = static_cast<int64_t>(t) * a.k_t + (static_cast<int64_t>(b) * a.N + n) * a.k_row + h * a.d;
      const int64_t rv = static_cast<int64_t>(t) * a.v_t + (static_cast<int64_t>(b) * a.N + n) * a.v_row + h * a.d;
      for (int dd = 0; dd < kMaxDim; ++dd) {
        const bool in = ok && dd < a.d;
        qs[n * kPitch + dd] = in ? bit_of(a.q[rq + dd]) : 0;
        ks[n * kPitch + dd] = in ? bit_of(a.k[rk + dd]) : 0;
        vt[dd * kPitch + n] = in ? bit_of(a.v[rv + dd]) : 0;
      }
    }
    __syncthreads();

    // ---- S = Q K^T ---------------------------------------------------------
#pragma unroll
    for (int ti = 0; ti < NT; ++ti) {
#pragma unroll
      for (int tj = 0; tj < NT; ++tj) {
        i32x16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
        for (int kk = 0; kk < kMaxDim / 32; ++kk) {
          const i32x4 fa = *reinterpret_cast<const i32x4*>(qs + (ti * 32 + r32) * kPitch + kk * 32 + g * 16);
          const i32x4 fb = *reinterpret_cast<const i32x4*>(ks + (tj * 32 + r32) * kPitch + kk * 32 + g * 16);
          acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, acc, 0, 0, 0);
        }
        // register e of lane l: row 8*(e/4) + 4*g + e%4, column l%32
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int i = ti * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
          const int j = tj * 32 + r32;
          ss[i * kPitch + j] = static_cast<int8_t>(acc[e]);
          if (a.s_counts && i < a.N && j < a.N)
            a.s_counts[((static_cast<int64_t>(t) * a.B * a.H + bh) * a.N + i) * a.N + j] = acc[e];
        }
      }
    }
    // tokens past N: S rows/cols are zero already (zero-padded Q, K); the
    // columns j >= 32*NT are never read.
    __syncthreads();

    // ---- O = S V and the LIF ---------------------------------------------------
#pragma unroll
    for (int ti = 0; ti < NT; ++ti) {
#pragma unroll
      for (int td = 0; td < DT; ++td) {
        i32x16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
        for (int kk = 0; kk < NT; ++kk) {
          const i32x4 fa = *reinterpret_cast<const i32x4*>(ss + (ti * 32 + r32) * kPitch + kk * 32 + g * 16);
          const i32x4 fb = *reinterpret_cast<const i32x4*>(vt + (td * 32 + r32) * kPitch + kk * 32 + g * 16);
          acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, acc, 0, 0, 0);
        }
        const int dd = td * 32 + r32;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int i = ti * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
          const float o = static_cast<float>(acc[e]);
          const float hm = __fadd_rn(__fmul_rn(a.decay, vm[ti][td][e]), __fmul_rn(a.in_scale, o));
          const bool s = hm >= a.vth;
          vm[ti][td][e] = s ? (a.soft_reset ? __fsub_rn(hm, a.vth) : a.v_reset) : hm;
          if (i < a.N && dd < a.d) {
            const int64_t row = static_cast<int64_t>(b) * a.N + i;
            a.out[static_cast<int64_t>(t) * a.o_t + row * a.o_row + h * a.d + dd] = s ? 0x3F80u : 0u;
            if (a.o_counts)
              a.o_counts[((static_cast<int64_t>(t) * a.B * a.H + bh) * a.N + i) * a.d + dd] = acc[e];
          }
        }
      }
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace snnk

using namespace snnk;

extern "C" int snnk_spike_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                    int64_t q_row, int64_t k_row, int64_t v_row,
                                    int64_t q_step, int64_t k_step, int64_t v_step,
                                    uint16_t* spikes_out, int64_t out_row, int64_t out_step,
                                    int32_t* s_counts, int32_t* o_counts,
                                    int64_t T, int64_t B, int64_t H, int64_t N, int64_t d,
                                    float decay, float in_scale, float v_threshold,
                                    float v_reset, int32_t soft_reset, void* stream) {
  if (T < 0 || B < 0 || H <= 0 || N < 0 || d <= 0) return SNNK_EINVAL;
  if (T == 0 || B == 0 || N == 0) return SNNK_OK;
  if (q == nullptr || k == nullptr || v == nullptr || spikes_out == nullptr) return SNNK_EINVAL;
  if (N > kMaxTok || d > kMaxDim) return SNNK_EUNSUPPORTED;
  if (q_row < H * d || k_row < H * d || v_row < H * d || out_row < H * d) return SNNK_EINVAL;
  if (B * H > 0x7FFFFFFFll) return SNNK_EUNSUPPORTED;
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v;
  a.q_row = q_row; a.k_row = k_row; a.v_row = v_row;
  a.q_t = q_step; a.k_t = k_step; a.v_t = v_step;
  a.out = spikes_out; a.o_row = out_row; a.o_t = out_step;
  a.s_counts = s_counts; a.o_counts = o_counts;
  a.T = static_cast<int>(T); a.B = static_cast<int>(B); a.H = static_cast<int>(H);
  a.N = static_cast<int>(N); a.d = static_cast<int>(d);
  a.decay = decay; a.in_scale = in_scale; a.vth = v_threshold; a.v_reset = v_reset;
  a.soft_reset = soft_reset ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nt = N > 32 ? 2 : 1, dt = d > 32 ? 2 : 1;
  if (nt == 1 && dt == 1) hipLaunchKernelGGL((ssa_attention_kernel<1, 1>), dim3(B * H), dim3(64), 0, s, a);
  else if (nt == 1) hipLaunchKernelGGL((ssa_attention_kernel<1, 2>), dim3(B * H), dim3(64), 0, s, a);
  else if (dt == 1) hipLaunchKernelGGL((ssa_attention_kernel<2, 1>), dim3(B * H), dim3(64), 0, s, a);
  else hipLaunchKernelGGL((ssa_attention_kernel<2, 2>), dim3(B * H), dim3(64), 0, s, a);
  return launch_status();
}
