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
  int o_vec;  // output rows and steps 8-byte aligned: 4 spikes per store
  int per_xcd;  // (batch, head) blocks per XCD
};

// Two words of bf16 pairs (4 elements) -> 4 bytes, 1 where the element is nonzero.
__device__ __forceinline__ uint32_t bytes4(uint32_t lo, uint32_t hi) {
  const uint32_t b0 = (lo & 0x7FFFu) ? 1u : 0u, b1 = (lo & 0x7FFF0000u) ? 1u : 0u;
  const uint32_t b2 = (hi & 0x7FFFu) ? 1u : 0u, b3 = (hi & 0x7FFF0000u) ? 1u : 0u;
  return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

// Block = 8 waves for one (batch, head).  Each of the 512 threads stages one
// 8-dim chunk of Q_t and of K_t and a 4-token x 2-dim patch of V_t; wave w
// computes S tile (w / NT, w % NT) when w < NT*NT and owns O tile
// (w / DT, w % DT) -- with its LIF membrane -- when w < NT*DT.  Both products
// are formed transposed (S^T = K Q^T, O^T = V^T S^T: the MFMA operands
// swapped) so that a lane's accumulator holds 4 consecutive columns of S and
// of O: one 4-byte LDS write per 4 entries of S and one 8-byte store per 4
// spikes of the output.
constexpr int kThreads = 512;
static_assert(kMaxTok * (kMaxDim / 8) == kThreads, "one Q/K chunk per thread");
static_assert((kMaxTok / 4) * (kMaxDim / 2) == kThreads, "one V patch per thread");

template <int NT, int DT>  // token tiles, dim tiles (32 each)
__global__ __launch_bounds__(kThreads) void ssa_attention_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t qs[kMaxTok * kPitch];
  __shared__ __attribute__((aligned(16))) int8_t ks[kMaxTok * kPitch];
  __shared__ __attribute__((aligned(16))) int8_t vt[kMaxDim * kPitch];  // [dim][token]
  __shared__ __attribute__((aligned(16))) int8_t ss[kMaxTok * kPitch];  // S as int8

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // Workgroups are dealt to the 8 XCDs round-robin by id; id -> (batch, head)
  // is remapped so that each XCD runs a contiguous range of heads.  The heads
  // of one batch then share an XCD's L2, which fetches each 128-byte line of
  // their token rows once (a head's d columns straddle lines that the
  // neighbouring heads also read).
  const int bh = (blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (bh >= a.B * a.H) return;
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
  // O^T accumulator of this lane: token oi*32 + r32, dims od*32 + 8*(e/4) + 4*g + e%4
  const int ti = oi * 32 + r32;
  uint16_t* ob = a.out + (row0 + ti) * a.o_row + h * a.d;
  float vm[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) vm[e] = 0.0f;

  // ---- staging of Q_t, K_t (row = token) and V_t^T (row = dim) as int8 ----
  // Q/K: thread = (token n, chunk c of 8 dims), one 16-byte load each.
  // V: thread = (4 tokens from 4*n4, dims 2p and 2p+1), four 4-byte loads that
  // become one 4-byte row segment of V^T per dim.  Padding tokens and dims
  // are zeros.  The loads of step t+1 are issued into registers before step
  // t's MFMAs, so only the first step waits for memory.
  const int qn = tid >> 3, qc = tid & 7;
  const int vp = tid & 31, vn4 = tid >> 5;
  const bool q_in = qn < a.N && qc * 8 < a.d;
  const bool v_in = 2 * vp < a.d;
  u32x4 rq, rk;
  uint32_t rv[4];
  auto load_step = [&](int t) {
    rq = rk = u32x4{0u, 0u, 0u, 0u};
    if (q_in) {
      rq = *reinterpret_cast<const u32x4*>(qb + t * a.q_t + qn * a.q_row + qc * 8);
      rk = *reinterpret_cast<const u32x4*>(kb + t * a.k_t + qn * a.k_row + qc * 8);
    }
    const uint16_t* vtp = vb + t * a.v_t + 2 * vp;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int n = 4 * vn4 + u;
      rv[u] = (v_in && n < a.N) ? *reinterpret_cast<const uint32_t*>(vtp + n * a.v_row) : 0u;
    }
  };
  auto store_step = [&]() {
    u32x2 bq, bk;
    bq[0] = bytes4(rq[0], rq[1]); bq[1] = bytes4(rq[2], rq[3]);
    bk[0] = bytes4(rk[0], rk[1]); bk[1] = bytes4(rk[2], rk[3]);
    *reinterpret_cast<u32x2*>(qs + qn * kPitch + qc * 8) = bq;
    *reinterpret_cast<u32x2*>(ks + qn * kPitch + qc * 8) = bk;
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      lo |= ((rv[u] & 0x7FFFu) ? 1u : 0u) << (8 * u);
      hi |= ((rv[u] & 0x7FFF0000u) ? 1u : 0u) << (8 * u);
    }
    *reinterpret_cast<uint32_t*>(vt + (2 * vp) * kPitch + 4 * vn4) = lo;
    *reinterpret_cast<uint32_t*>(vt + (2 * vp + 1) * kPitch + 4 * vn4) = hi;
  };

  load_step(0);
  for (int t = 0; t < a.T; ++t) {
    store_step();
    __syncthreads();
    if (t + 1 < a.T) load_step(t + 1);

    // ---- S^T = K Q^T (one 32x32 tile per wave) ------------------------------
    if (has_s) {
      i32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
      for (int kk = 0; kk < kMaxDim / 32; ++kk) {
        const i32x4 fk = *reinterpret_cast<const i32x4*>(ks + (sj * 32 + r32) * kPitch + kk * 32 + g * 16);
        const i32x4 fq = *reinterpret_cast<const i32x4*>(qs + (si * 32 + r32) * kPitch + kk * 32 + g * 16);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fk, fq, acc, 0, 0, 0);
      }
      // register e of lane l: S[i][j] with i = si*32 + l%32 (query) and
      // j = sj*32 + 8*(e/4) + 4*g + e%4 (key): 4 consecutive j per e/4
      const int i = si * 32 + r32;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const uint32_t w = (static_cast<uint32_t>(acc[4 * e4]) & 0xFFu) |
                           ((static_cast<uint32_t>(acc[4 * e4 + 1]) & 0xFFu) << 8) |
                           ((static_cast<uint32_t>(acc[4 * e4 + 2]) & 0xFFu) << 16) |
                           (static_cast<uint32_t>(acc[4 * e4 + 3]) << 24);
        *reinterpret_cast<uint32_t*>(ss + i * kPitch + sj * 32 + 8 * e4 + 4 * g) = w;
      }
      if (a.s_counts) {
        int32_t* sc = a.s_counts + ((static_cast<int64_t>(t) * a.B * a.H + bh) * a.N) * a.N;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int j = sj * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
          if (i < a.N && j < a.N) sc[i * a.N + j] = acc[e];
        }
      }
    }
    __syncthreads();

    // ---- O^T = V^T S^T and the LIF (one 32x32 tile per wave) -------------------
    if (has_o) {
      i32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
      for (int kk = 0; kk < NT; ++kk) {
        const i32x4 fv = *reinterpret_cast<const i32x4*>(vt + (od * 32 + r32) * kPitch + kk * 32 + g * 16);
        const i32x4 fs = *reinterpret_cast<const i32x4*>(ss + (oi * 32 + r32) * kPitch + kk * 32 + g * 16);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fv, fs, acc, 0, 0, 0);
      }
      uint16_t* ot = ob + t * a.o_t;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        uint32_t spk[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = 4 * e4 + u;
          const float hm = __fadd_rn(__fmul_rn(a.decay, vm[e]), __fmul_rn(a.in_scale, static_cast<float>(acc[e])));
          const bool sp = hm >= a.vth;
          vm[e] = sp ? (a.soft_reset ? __fsub_rn(hm, a.vth) : a.v_reset) : hm;
          spk[u] = sp ? 0x3F80u : 0u;
        }
        // 4 dims from dd0; d % 8 == 0, so they are all in range when dd0 is
        const int dd0 = od * 32 + 8 * e4 + 4 * g;
        if (ti < a.N && dd0 < a.d) {
          if (a.o_vec) {
            *reinterpret_cast<u32x2*>(ot + dd0) = u32x2{spk[0] | (spk[1] << 16), spk[2] | (spk[3] << 16)};
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) ot[dd0 + u] = static_cast<uint16_t>(spk[u]);
          }
        }
      }
      if (a.o_counts) {
        int32_t* oc = a.o_counts + ((static_cast<int64_t>(t) * a.B * a.H + bh) * a.N) * a.d;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int dd = od * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
          if (ti < a.N && dd < a.d) oc[ti * a.d + dd] = acc[e];
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
  a.o_vec = aligned(spikes_out, 8) && out_row % 4 == 0 && out_step % 4 == 0;
  a.per_xcd = static_cast<int>((B * H + 7) / 8);
  const dim3 grid(static_cast<unsigned>(a.per_xcd) * 8u);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nt = N > 32 ? 2 : 1, dt = d > 32 ? 2 : 1;
  if (nt == 1 && dt == 1) hipLaunchKernelGGL((ssa_attention_kernel<1, 1>), grid, dim3(kThreads), 0, s, a);
  else if (nt == 1) hipLaunchKernelGGL((ssa_attention_kernel<1, 2>), grid, dim3(kThreads), 0, s, a);
  else if (dt == 1) hipLaunchKernelGGL((ssa_attention_kernel<2, 1>), grid, dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((ssa_attention_kernel<2, 2>), grid, dim3(kThreads), 0, s, a);
  return launch_status();
}
