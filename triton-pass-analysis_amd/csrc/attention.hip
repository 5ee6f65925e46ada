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
// One block per (batch, head).  Per step t the block stages Q_t, K_t and
// V_t^T of its head in LDS as int8 (read from memory one step ahead; zero
// padded to 64 tokens x 64 dims; d % 8 == 0, rows 16-byte aligned), computes
// S = Q K^T into accumulators, writes S to LDS as int8 (0 <= S <= d <= 64),
// computes O = S V, and runs the LIF v = decay*v + in_scale*O on O in
// registers; the membrane of every (token, dim) stays in the same lane of the
// same wave for all T steps.
#include "snnk_common.h"

namespace snnk {

// Linear-order path for more than 64 tokens or dims (attention_linear.hip).
int spike_attention_linear(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           int64_t q_row, int64_t k_row, int64_t v_row, int64_t q_step,
                           int64_t k_step, int64_t v_step, uint16_t* spikes_out,
                           int64_t out_row, int64_t out_step, int32_t* o_counts, int64_t T,
                           int64_t B, int64_t H, int64_t N, int64_t d, float decay,
                           float in_scale, float v_threshold, float v_reset, int32_t soft_reset,
                           hipStream_t s);

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

// Nonzero test of the two bf16 in a word, sign ignored: bit 15 (31) of the
// result is set iff the low (high) element is nonzero -- each 15-bit
// magnitude plus 0x7FFF reaches 0x8000 iff it is at least 1 and stays below
// 0x10000, so no carry crosses the halves.  Bits below the flags are junk.
__device__ __forceinline__ uint32_t nz_pairs(uint32_t w) { return (w & 0x7FFF7FFFu) + 0x7FFF7FFFu; }

// Four flags at bit 7 of the bytes that `sel` picks from {hi:lo} -> four
// bytes 0/1 (v_perm_b32: selector byte k picks byte sel_k of the 8-byte
// value whose low word is lo).
__device__ __forceinline__ uint32_t flag_bytes(uint32_t hi, uint32_t lo, uint32_t sel) {
  return (__builtin_amdgcn_perm(hi, lo, sel) >> 7) & 0x01010101u;
}

// Block = 8 waves for one (batch, head), in two roles so that no wave both
// waits for loads and has stores in flight (one vmcnt counts both):
//  * waves 4..7 stage: each of their 256 threads turns two 8-dim chunks of
//    Q_t and K_t and two 4-token x 2-dim patches of V_t into int8 rows of a
//    double-buffered LDS stage (loads one step ahead), and waves 4..4+NT*NT-1
//    compute S tile (w-4)/NT, (w-4)%NT;
//  * waves 0..NT*DT-1 own O tile (w / DT, w % DT) with its LIF membrane and
//    write the output spikes.
// Per step t two barriers: [stage t+1 | O_t, LIF, stores] then [S_{t+1}].
// Both products are formed transposed (S^T = K Q^T, O^T = V^T S^T: the MFMA
// operands swapped) so that a lane's accumulator holds 4 consecutive columns
// of S and of O: one 4-byte LDS write per 4 entries of S and one 8-byte store
// per 4 spikes of the output.
constexpr int kThreads = 512;
constexpr int kStagers = 256;                  // threads of waves 4..7
constexpr int kStage = kMaxTok * kPitch;       // bytes of one staged int8 matrix
constexpr int kRsrcWord3 = 0x00020000;         // raw buffer, 32-bit data format
static_assert(kMaxTok == kMaxDim, "Q, K, V^T and S share one staging size");
static_assert(kMaxTok * (kMaxDim / 8) == 2 * kStagers, "two Q/K chunks per stager");
static_assert((kMaxTok / 4) * (kMaxDim / 2) == 2 * kStagers, "two V patches per stager");

template <int NT, int DT, bool SR>  // token tiles, dim tiles (32 each), soft reset
__global__ __launch_bounds__(kThreads) void ssa_attention_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t qs[2 * kStage];
  __shared__ __attribute__((aligned(16))) int8_t ks[2 * kStage];
  __shared__ __attribute__((aligned(16))) int8_t vt[2 * kStage];  // [dim][token]
  __shared__ __attribute__((aligned(16))) int8_t ss[2 * kStage];  // S as int8

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

  const bool stager = wave >= 4;
  const bool has_s = stager && wave - 4 < NT * NT;
  const int si = (wave - 4) / NT, sj = (wave - 4) % NT;
  const bool has_o = wave < NT * DT;
  const int oi = wave / DT, od = wave % DT;
  // O^T accumulator of this lane: token oi*32 + r32, dims od*32 + 8*(e/4) + 4*g + e%4
  const int ti = oi * 32 + r32;
  uint16_t* ob = a.out + (row0 + ti) * a.o_row + h * a.d;
  float vm[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) vm[e] = 0.0f;

  // ---- staging of Q_t, K_t (row = token) and V_t^T (row = dim) as int8 ----
  // item m of stager st: Q/K chunk (token n = c/8, dims 8*(c%8)..+7) and V
  // patch (tokens 4*(c/32)..+3, dims 2*(c%32), +1) for c = st + 256*m.
  // Padding tokens and dims are zeros.
  const int st = tid - (kThreads - kStagers);
  // Loads go through buffer descriptors based at the step's slice, with a
  // per-thread byte offset fixed for the whole kernel; padding tokens and
  // dims get an offset past the descriptor's range, which reads zeros.
  constexpr uint32_t kOutside = 0x80000000u;  // > kRecords
  constexpr int kRecords = 0x7FFFFFFF;
  uint32_t qoff[2], koff[2], voff[2][4];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int c = st + kStagers * m;
    const int qn = c >> 3, qc = c & 7;
    const bool in = qn < a.N && qc * 8 < a.d;
    qoff[m] = in ? static_cast<uint32_t>((qn * a.q_row + qc * 8) * 2) : kOutside;
    koff[m] = in ? static_cast<uint32_t>((qn * a.k_row + qc * 8) * 2) : kOutside;
    const int vp = c & 31, vn4 = c >> 5;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int n = 4 * vn4 + x;
      voff[m][x] = (2 * vp < a.d && n < a.N) ? static_cast<uint32_t>((n * a.v_row + 2 * vp) * 2) : kOutside;
    }
  }
  u32x4 rq[2], rk[2];
  uint32_t rv[2][4];
  auto load_step = [&](int t) {
    const __amdgpu_buffer_rsrc_t qr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(qb + t * a.q_t), 0, kRecords, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kb + t * a.k_t), 0, kRecords, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vb + t * a.v_t), 0, kRecords, kRsrcWord3);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const i32x4 q4 = __builtin_amdgcn_raw_buffer_load_b128(qr, qoff[m], 0, 0);
      const i32x4 k4 = __builtin_amdgcn_raw_buffer_load_b128(kr, koff[m], 0, 0);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        rq[m][w] = static_cast<uint32_t>(q4[w]);
        rk[m][w] = static_cast<uint32_t>(k4[w]);
      }
#pragma unroll
      for (int x = 0; x < 4; ++x) rv[m][x] = __builtin_amdgcn_raw_buffer_load_b32(vr, voff[m][x], 0, 0);
    }
  };
  auto store_step = [&](int buf) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int c = st + kStagers * m;
      const int qn = c >> 3, qc = c & 7;
      // dims 0..3 from words 0, 1 and dims 4..7 from words 2, 3: flags in bytes 1, 3
      const u32x2 bq{flag_bytes(nz_pairs(rq[m][1]), nz_pairs(rq[m][0]), 0x07050301u),
                     flag_bytes(nz_pairs(rq[m][3]), nz_pairs(rq[m][2]), 0x07050301u)};
      const u32x2 bk{flag_bytes(nz_pairs(rk[m][1]), nz_pairs(rk[m][0]), 0x07050301u),
                     flag_bytes(nz_pairs(rk[m][3]), nz_pairs(rk[m][2]), 0x07050301u)};
      *reinterpret_cast<u32x2*>(qs + buf * kStage + qn * kPitch + qc * 8) = bq;
      *reinterpret_cast<u32x2*>(ks + buf * kStage + qn * kPitch + qc * 8) = bk;
      // token x's word holds dims 2p (byte 1 flag) and 2p+1 (byte 3 flag)
      const uint32_t x01 = __builtin_amdgcn_perm(nz_pairs(rv[m][1]), nz_pairs(rv[m][0]), 0x07030501u);
      const uint32_t x23 = __builtin_amdgcn_perm(nz_pairs(rv[m][3]), nz_pairs(rv[m][2]), 0x07030501u);
      const int vp = c & 31, vn4 = c >> 5;
      *reinterpret_cast<uint32_t*>(vt + buf * kStage + (2 * vp) * kPitch + 4 * vn4) = flag_bytes(x23, x01, 0x05040100u);
      *reinterpret_cast<uint32_t*>(vt + buf * kStage + (2 * vp + 1) * kPitch + 4 * vn4) = flag_bytes(x23, x01, 0x07060302u);
    }
  };

  // ---- S_t^T = K_t Q_t^T (one 32x32 tile per S wave) ---------------------------
  auto s_step = [&](int t) {
    const int buf = t & 1;
    i32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
    for (int kk = 0; kk < kMaxDim / 32; ++kk) {
      const i32x4 fk = *reinterpret_cast<const i32x4*>(ks + buf * kStage + (sj * 32 + r32) * kPitch + kk * 32 + g * 16);
      const i32x4 fq = *reinterpret_cast<const i32x4*>(qs + buf * kStage + (si * 32 + r32) * kPitch + kk * 32 + g * 16);
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
      *reinterpret_cast<uint32_t*>(ss + buf * kStage + i * kPitch + sj * 32 + 8 * e4 + 4 * g) = w;
    }
    if (a.s_counts) {
      int32_t* sc = a.s_counts + ((static_cast<int64_t>(t) * a.B * a.H + bh) * a.N) * a.N;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int j = sj * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
        if (i < a.N && j < a.N) sc[i * a.N + j] = acc[e];
      }
    }
  };

  if (stager) {
    load_step(0);
    store_step(0);
    if (a.T > 1) load_step(1);
  }
  __syncthreads();
  if (has_s) s_step(0);
  __syncthreads();
  for (int t = 0; t < a.T; ++t) {
    if (stager) {
      if (t + 1 < a.T) {
        store_step((t + 1) & 1);
        if (t + 2 < a.T) load_step(t + 2);
      }
    } else if (has_o) {
      // ---- O_t^T = V_t^T S_t^T and the LIF (one 32x32 tile per O wave) -------
      const int buf = t & 1;
      i32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
      for (int kk = 0; kk < NT; ++kk) {
        const i32x4 fv = *reinterpret_cast<const i32x4*>(vt + buf * kStage + (od * 32 + r32) * kPitch + kk * 32 + g * 16);
        const i32x4 fs = *reinterpret_cast<const i32x4*>(ss + buf * kStage + (oi * 32 + r32) * kPitch + kk * 32 + g * 16);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fv, fs, acc, 0, 0, 0);
      }
      uint16_t* ot = ob + t * a.o_t;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        uint32_t spk[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const int e = 4 * e4 + x;
          const float hm = __fadd_rn(__fmul_rn(a.decay, vm[e]), __fmul_rn(a.in_scale, static_cast<float>(acc[e])));
          const bool sp = hm >= a.vth;
          vm[e] = sp ? (SR ? __fsub_rn(hm, a.vth) : a.v_reset) : hm;
          spk[x] = sp ? 0x3F80u : 0u;
        }
        // 4 dims from dd0; d % 8 == 0, so they are all in range when dd0 is
        const int dd0 = od * 32 + 8 * e4 + 4 * g;
        if (ti < a.N && dd0 < a.d) {
          if (a.o_vec) {
            *reinterpret_cast<u32x2*>(ot + dd0) = u32x2{spk[0] | (spk[1] << 16), spk[2] | (spk[3] << 16)};
          } else {
#pragma unroll
            for (int x = 0; x < 4; ++x) ot[dd0 + x] = static_cast<uint16_t>(spk[x]);
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
    if (has_s && t + 1 < a.T) s_step(t + 1);
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
  if (d % 8 != 0) return SNNK_EUNSUPPORTED;
  // more than 64 tokens or dims: the linear order Q (K^T V), which has no S
  const bool linear = N > kMaxTok || d > kMaxDim;
  if (linear && s_counts != nullptr) return SNNK_EUNSUPPORTED;
  // 16-byte chunk loads: every row start and head offset on a 16-byte boundary
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || q_row % 8 || k_row % 8 ||
      v_row % 8 || q_step % 8 || k_step % 8 || v_step % 8)
    return SNNK_EALIGN;
  if (q_row < H * d || k_row < H * d || v_row < H * d || out_row < H * d) return SNNK_EINVAL;
  if (B * H > 0x7FFFFFFFll) return SNNK_EUNSUPPORTED;
  // byte offsets of a step's token rows stay below 2^31 (buffer offsets)
  if (std::max(q_row, std::max(k_row, v_row)) >= (int64_t{1} << 23)) return SNNK_EUNSUPPORTED;
  if (linear)
    return spike_attention_linear(q, k, v, q_row, k_row, v_row, q_step, k_step, v_step,
                                  spikes_out, out_row, out_step, o_counts, T, B, H, N, d, decay,
                                  in_scale, v_threshold, v_reset, soft_reset,
                                  static_cast<hipStream_t>(stream));
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
  auto launch = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, a); };
  if (soft_reset) {
    if (nt == 1 && dt == 1) launch(ssa_attention_kernel<1, 1, true>);
    else if (nt == 1) launch(ssa_attention_kernel<1, 2, true>);
    else if (dt == 1) launch(ssa_attention_kernel<2, 1, true>);
    else launch(ssa_attention_kernel<2, 2, true>);
  } else {
    if (nt == 1 && dt == 1) launch(ssa_attention_kernel<1, 1, false>);
    else if (nt == 1) launch(ssa_attention_kernel<1, 2, false>);
    else if (dt == 1) launch(ssa_attention_kernel<2, 1, false>);
    else launch(ssa_attention_kernel<2, 2, false>);
  }
  return launch_status();
}
