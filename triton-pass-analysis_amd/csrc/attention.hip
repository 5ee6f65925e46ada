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
// One block per (batch, head).  Per step t the block stages Q_t,
// K_t and V_t^T of its head in LDS as int8 (read from memory one step ahead) (zero padded to 64 tokens x 64
// dims; d % 8 == 0, rows 16-byte aligned), computes S = Q K^T into accumulators, writes S to LDS as int8
// (0 <= S <= d <= 64), computes O = S V, and runs the LIF
// v = decay*v + in_scale*O on O in registers; the membrane of every
// (token, dim) stays in the same lane of the same wave for all T steps.
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

// Two words of bf16 pairs (4 elements) -> 4 bytes, 1 where the element is nonzero.
__device__ __forceinline__ uint32_t bytes4(uint32_t lo, uint32_t hi) {
  const uint32_t b0 = (lo & 0x7FFFu) ? 1u : 0u, b1 = (lo & 0x7FFF0000u) ? 1u : 0u;
  const uint32_t b2 = (hi & 0x7FFFu) ? 1u : 0u, b3 = (hi & 0x7FFF0000u) ? 1u : 0u;
  return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

// Block = 4 waves for one (batch, head).  Staging is shared by the 256
// threads; wave w computes S tile (w / NT, w % NT) when w < NT*NT and owns
// O tile (w / DT, w % DT) -- with its LIF membrane -- when w < NT*DT.
template <int NT, int DT>  // token tiles, dim tiles (32 each)
__global__ __launch_bounds__(256) void ssa_attention_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t qs[kMaxTok * kPitch];
  __shared__ __attribute__((aligned(16))) int8_t ks[kMaxTok * kPitch];
  __shared__ __attribute__((aligned(16))) int8_t vt[kMaxDim * kPitch];  // [dim][token]
  __shared__ __attribute__((aligned(16))) int8_t ss[kMaxTok * kPitch];  // S as int8

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - b * a.H;
  const int r32 = lane & 31, g = lane >> 5;
  // this block's (batch, head) slice: token row 0, column h*d
  const int64_t row0 = static_cast<int64_t>(b) * a.N;
  const uint16_t* qb = a.q + row0 * a.q_row + h * a.d;
  const uint16_t* kb = a.k + row0 * a.k_row + h * a.d;
  const uint16_t* vb = a.v + row0 * a.v_row + h * a.d;

  const bool has_s = wave < NT * NT;
  const int si = wave / NT, sj = wave % NT;
  const bool has_o = wave < NT * DT;
  const int oi = wave / DT, od = wave % DT;
  const int dd = od * 32 + r32;
  uint16_t* ob = a.out + row0 * a.o_row + h * a.d + dd;
  float vm[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) vm[e] = 0.0f;

  // ---- staging of Q_t, K_t (row = token) and V_t^T (row = dim) as int8 ----
  // 64 tokens x 8 chunks of 8 dims per tensor; consecutive threads walk along
  // a token row with 16-byte loads; padding rows / dims are zeros.  The loads
  // of step t+1 are issued into registers before step t's MFMAs, so only the
  // first step waits for memory.
  u32x4 rq[2], rk[2], rv[2];
  auto load_step = [&](int t) {
    const uint16_t* qt = qb + t * a.q_t;
    const uint16_t* kt = kb + t * a.k_t;
    const uint16_t* vtp = vb + t * a.v_t;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int ci = tid + 256 * m;
      const int n = ci >> 3, c = ci & 7;
      rq[m] = rk[m] = rv[m] = u32x4{0u, 0u, 0u, 0u};
      if (n < a.N && c * 8 < a.d) {
        rq[m] = *reinterpret_cast<const u32x4*>(qt + n * a.q_row + c * 8);
        rk[m] = *reinterpret_cast<const u32x4*>(kt + n * a.k_row + c * 8);
        rv[m] = *reinterpret_cast<const u32x4*>(vtp + n * a.v_row + c * 8);
      }
    }
  };
  auto store_step = [&]() {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int ci = tid + 256 * m;
      const int n = ci >> 3, c = ci & 7;
      u32x2 bq, bk;
      bq[0] = bytes4(rq[m][0], rq[m][1]); bq[1] = bytes4(rq[m][2], rq[m][3]);
      bk[0] = bytes4(rk[m][0], rk[m][1]); bk[1] = bytes4(rk[m][2], rk[m][3]);
      *reinterpret_cast<u32x2*>(qs + n * kPitch + c * 8) = bq;
      *reinterpret_cast<u32x2*>(ks + n * kPitch + c * 8) = bk;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t w = rv[m][e >> 1] >> (16 * (e & 1));
        vt[(c * 8 + e) * kPitch + n] = (w & 0x7FFFu) ? 1 : 0;
      }
    }
  };

  load_step(0);
  for (int t = 0; t < a.T; ++t) {
    store_step();
    __syncthreads();
    if (t + 1 < a.T) load_step(t + 1);

    // ---- S = Q K^T (one 32x32 tile per wave) --------------------------------
    if (has_s) {
      i32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
      for (int kk = 0; kk < kMaxDim / 32; ++kk) {
        const i32x4 fa = *reinterpret_cast<const i32x4*>(qs + (si * 32 + r32) * kPitch + kk * 32 + g * 16);
        const i32x4 fb = *reinterpret_cast<const i32x4*>(ks + (sj * 32 + r32) * kPitch + kk * 32 + g * 16);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, acc, 0, 0, 0);
      }
      // register e of lane l: row 8*(e/4) + 4*g + e%4, column l%32
      const int j = sj * 32 + r32;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = si * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
        ss[i * kPitch + j] = static_cast<int8_t>(acc[e]);
      }
      if (a.s_counts) {
        int32_t* sc = a.s_counts + ((static_cast<int64_t>(t) * a.B * a.H + bh) * a.N) * a.N;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int i = si * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
          if (i < a.N && j < a.N) sc[i * a.N + j] = acc[e];
        }
      }
    }
    __syncthreads();

    // ---- O = S V and the LIF (one 32x32 tile per wave) --------------------------
    if (has_o) {
      i32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
      for (int kk = 0; kk < NT; ++kk) {
        const i32x4 fa = *reinterpret_cast<const i32x4*>(ss + (oi * 32 + r32) * kPitch + kk * 32 + g * 16);
        const i32x4 fb = *reinterpret_cast<const i32x4*>(vt + (od * 32 + r32) * kPitch + kk * 32 + g * 16);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, acc, 0, 0, 0);
      }
      uint16_t* ot = ob + t * a.o_t;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = oi * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
        const float hm = __fadd_rn(__fmul_rn(a.decay, vm[e]), __fmul_rn(a.in_scale, static_cast<float>(acc[e])));
        const bool sp = hm >= a.vth;
        vm[e] = sp ? (a.soft_reset ? __fsub_rn(hm, a.vth) : a.v_reset) : hm;
        if (i < a.N && dd < a.d) ot[i * a.o_row] = sp ? 0x3F80u : 0u;
      }
      if (a.o_counts) {
        int32_t* oc = a.o_counts + ((static_cast<int64_t>(t) * a.B * a.H + bh) * a.N) * a.d;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int i = oi * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
          if (i < a.N && dd < a.d) oc[i * a.d + dd] = acc[e];
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
  if (N > kMaxTok || d > kMaxDim || d % 8 != 0) return SNNK_EUNSUPPORTED;
  // 16-byte chunk loads: every row start and head offset on a 16-byte boundary
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || q_row % 8 || k_row % 8 ||
      v_row % 8 || q_step % 8 || k_step % 8 || v_step % 8)
    return SNNK_EALIGN;
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
  if (nt == 1 && dt == 1) hipLaunchKernelGGL((ssa_attention_kernel<1, 1>), dim3(B * H), dim3(256), 0, s, a);
  else if (nt == 1) hipLaunchKernelGGL((ssa_attention_kernel<1, 2>), dim3(B * H), dim3(256), 0, s, a);
  else if (dt == 1) hipLaunchKernelGGL((ssa_attention_kernel<2, 1>), dim3(B * H), dim3(256), 0, s, a);
  else hipLaunchKernelGGL((ssa_attention_kernel<2, 2>), dim3(B * H), dim3(256), 0, s, a);
  return launch_status();
}
