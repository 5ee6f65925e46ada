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
  // packed spikes (PK kernels): q, k, v and out are uint32 words of LSB-first
  // bits; head h of q, k, v starts at bit h*hbits of a row (a multiple of 8,
  // so 8 dims never straddle a word), head h of out at word h*ohw; row and
  // step strides count words
  int hbits, ohw;
};

// 8 spikes (bits of b, LSB first) -> 8 int8 0/1: each nibble times
// 0x00204081 puts its bit i at bit 8*i + ... with no overlap, and the mask
// keeps bit 0 of every byte.
__device__ __forceinline__ u32x2 bits_to_bytes8(uint32_t b) {
  return u32x2{((b & 0xFu) * 0x00204081u) & 0x01010101u, (((b >> 4) & 0xFu) * 0x00204081u) & 0x01010101u};
}

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

// token tiles, dim tiles (32 each), soft reset, packed spikes in and out
template <int NT, int DT, bool SR, bool PK>
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
  // the block's first token row (packed: the head's bit offset goes into the
  // per-thread offsets) or its head's first element (bf16)
  const int64_t hcol = PK ? 0 : static_cast<int64_t>(h) * a.d;
  const int hbit0 = PK ? h * a.hbits : 0;
  const uint16_t* qb = PK ? reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint32_t*>(a.q) + row0 * a.q_row)
                          : a.q + row0 * a.q_row + hcol;
  const uint16_t* kb = PK ? reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint32_t*>(a.k) + row0 * a.k_row)
                          : a.k + row0 * a.k_row + hcol;
  const uint16_t* vb = PK ? reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint32_t*>(a.v) + row0 * a.v_row)
                          : a.v + row0 * a.v_row + hcol;
  constexpr int kElem = PK ? 4 : 2;  // bytes per stride unit

  const bool stager = wave >= 4;
  const bool has_s = stager && wave - 4 < NT * NT;
  const int si = (wave - 4) / NT, sj = (wave - 4) % NT;
  const bool has_o = wave < NT * DT;
  const int oi = wave / DT, od = wave % DT;
  // O^T accumulator of this lane: token oi*32 + r32, dims od*32 + 8*(e/4) + 4*g + e%4
  const int ti = oi * 32 + r32;
  uint16_t* ob = a.out + (row0 + ti) * a.o_row + h * a.d;  // (bf16 output)
  uint32_t* obw = reinterpret_cast<uint32_t*>(a.out) + (row0 + ti) * a.o_row +
                  static_cast<int64_t>(h) * a.ohw;  // (packed)
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
  uint32_t qsh[2], vsh[2];  // packed: bit position of the chunk / dim pair in its word
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int c = st + kStagers * m;
    const int qn = c >> 3, qc = c & 7;
    const bool in = qn < a.N && qc * 8 < a.d;
    // bf16: the chunk's 8 elements; packed: the word holding its 8 bits
    const int qcol = PK ? (hbit0 + 8 * qc) >> 5 : qc * 8;
    qsh[m] = static_cast<uint32_t>((hbit0 + 8 * qc) & 31);
    qoff[m] = in ? static_cast<uint32_t>((qn * a.q_row + qcol) * kElem) : kOutside;
    koff[m] = in ? static_cast<uint32_t>((qn * a.k_row + qcol) * kElem) : kOutside;
    const int vp = c & 31, vn4 = c >> 5;
    const int vcol = PK ? (hbit0 + 2 * vp) >> 5 : 2 * vp;
    vsh[m] = static_cast<uint32_t>((hbit0 + 2 * vp) & 31);
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int n = 4 * vn4 + x;
      voff[m][x] = (2 * vp < a.d && n < a.N) ? static_cast<uint32_t>((n * a.v_row + vcol) * kElem) : kOutside;
    }
  }
  u32x4 rq[2], rk[2];
  uint32_t rv[2][4];
  auto load_step = [&](int t) {
    const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(reinterpret_cast<const unsigned char*>(qb) + t * a.q_t * kElem), 0, kRecords, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(reinterpret_cast<const unsigned char*>(kb) + t * a.k_t * kElem), 0, kRecords, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(reinterpret_cast<const unsigned char*>(vb) + t * a.v_t * kElem), 0, kRecords, kRsrcWord3);
    if constexpr (PK) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        rq[m][0] = __builtin_amdgcn_raw_buffer_load_b32(qr, qoff[m], 0, 0);
        rk[m][0] = __builtin_amdgcn_raw_buffer_load_b32(kr, koff[m], 0, 0);
#pragma unroll
        for (int x = 0; x < 4; ++x) rv[m][x] = __builtin_amdgcn_raw_buffer_load_b32(vr, voff[m][x], 0, 0);
      }
      return;
    }
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
    if constexpr (PK) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int c = st + kStagers * m;
        const int qn = c >> 3, qc = c & 7;
        // the chunk's 8 dims sit at bit qsh of its word
        *reinterpret_cast<u32x2*>(qs + buf * kStage + qn * kPitch + qc * 8) =
            bits_to_bytes8(rq[m][0] >> qsh[m]);
        *reinterpret_cast<u32x2*>(ks + buf * kStage + qn * kPitch + qc * 8) =
            bits_to_bytes8(rk[m][0] >> qsh[m]);
        // dims 2p, 2p+1 are bits vsh, vsh+1 of each token's word
        const int vp = c & 31, vn4 = c >> 5;
        const uint32_t sh = vsh[m];
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          w0 |= ((rv[m][x] >> sh) & 1u) << (8 * x);
          w1 |= ((rv[m][x] >> (sh + 1)) & 1u) << (8 * x);
        }
        *reinterpret_cast<uint32_t*>(vt + buf * kStage + (2 * vp) * kPitch + 4 * vn4) = w0;
        *reinterpret_cast<uint32_t*>(vt + buf * kStage + (2 * vp + 1) * kPitch + 4 * vn4) = w1;
      }
      return;
    }
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
      // packed: this lane's spikes at bit 8*e4 + 4*g + x of word od
      uint32_t bits = 0;
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
          if constexpr (PK) bits |= (sp && od * 32 + 8 * e4 + 4 * g + x < a.d ? 1u : 0u) << (8 * e4 + 4 * g + x);
        }
        if constexpr (!PK) {
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
      }
      if constexpr (PK) {
        // the two lane halves hold the word's other 16 bits (lane ^ 32)
        bits |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(bits), 32));
        if (g == 0 && ti < a.N && od * 32 < a.d) obw[t * a.o_t + od] = bits;
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

// Launch the core for args a (nt / dt: 32-token / 32-dim tiles).
template <bool PK>
int launch_core(const AttnArgs& a, int nt, int dt, bool soft, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.per_xcd) * 8u);
  auto launch = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, a); };
  if (soft) {
    if (nt == 1 && dt == 1) launch(ssa_attention_kernel<1, 1, true, PK>);
    else if (nt == 1) launch(ssa_attention_kernel<1, 2, true, PK>);
    else if (dt == 1) launch(ssa_attention_kernel<2, 1, true, PK>);
    else launch(ssa_attention_kernel<2, 2, true, PK>);
  } else {
    if (nt == 1 && dt == 1) launch(ssa_attention_kernel<1, 1, false, PK>);
    else if (nt == 1) launch(ssa_attention_kernel<1, 2, false, PK>);
    else if (dt == 1) launch(ssa_attention_kernel<2, 1, false, PK>);
    else launch(ssa_attention_kernel<2, 2, false, PK>);
  }
  return launch_status();
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
  return launch_core<false>(a, N > 32 ? 2 : 1, d > 32 ? 2 : 1, soft_reset != 0,
                            static_cast<hipStream_t>(stream));
}

extern "C" int snnk_spike_attention_packed(const uint32_t* q, const uint32_t* k, const uint32_t* v,
                                           int64_t q_row, int64_t k_row, int64_t v_row,
                                           int64_t q_step, int64_t k_step, int64_t v_step,
                                           int64_t in_head_bits, uint32_t* spikes_out,
                                           int64_t out_row, int64_t out_step,
                                           int64_t out_head_words,
                                           int32_t* s_counts, int32_t* o_counts,
                                           int64_t T, int64_t B, int64_t H, int64_t N, int64_t d,
                                           float decay, float in_scale, float v_threshold,
                                           float v_reset, int32_t soft_reset, void* stream) {
  if (T < 0 || B < 0 || H <= 0 || N < 0 || d <= 0) return SNNK_EINVAL;
  if (T == 0 || B == 0 || N == 0) return SNNK_OK;
  if (q == nullptr || k == nullptr || v == nullptr || spikes_out == nullptr) return SNNK_EINVAL;
  if (d % 8 != 0 || N > kMaxTok || d > kMaxDim) return SNNK_EUNSUPPORTED;
  if (in_head_bits < d || in_head_bits % 8 != 0 || out_head_words < (d + 31) / 32)
    return SNNK_EINVAL;
  if (!aligned(q, 4) || !aligned(k, 4) || !aligned(v, 4) || !aligned(spikes_out, 4))
    return SNNK_EALIGN;
  const int64_t need_in = (H * in_head_bits + 31) / 32;
  if (q_row < need_in || k_row < need_in || v_row < need_in || out_row < H * out_head_words)
    return SNNK_EINVAL;
  if (H * in_head_bits >= (int64_t{1} << 30)) return SNNK_EUNSUPPORTED;
  if (B * H > 0x7FFFFFFFll) return SNNK_EUNSUPPORTED;
  // byte offsets of a step's token rows stay below 2^31 (buffer offsets)
  if (std::max(q_row, std::max(k_row, v_row)) * kMaxTok * 4 >= (int64_t{1} << 31))
    return SNNK_EUNSUPPORTED;
  AttnArgs a{};
  a.q = reinterpret_cast<const uint16_t*>(q);
  a.k = reinterpret_cast<const uint16_t*>(k);
  a.v = reinterpret_cast<const uint16_t*>(v);
  a.q_row = q_row; a.k_row = k_row; a.v_row = v_row;
  a.q_t = q_step; a.k_t = k_step; a.v_t = v_step;
  a.out = reinterpret_cast<uint16_t*>(spikes_out); a.o_row = out_row; a.o_t = out_step;
  a.s_counts = s_counts; a.o_counts = o_counts;
  a.T = static_cast<int>(T); a.B = static_cast<int>(B); a.H = static_cast<int>(H);
  a.N = static_cast<int>(N); a.d = static_cast<int>(d);
  a.decay = decay; a.in_scale = in_scale; a.vth = v_threshold; a.v_reset = v_reset;
  a.soft_reset = soft_reset ? 1 : 0;
  a.hbits = static_cast<int>(in_head_bits);
  a.ohw = static_cast<int>(out_head_words);
  a.per_xcd = static_cast<int>((B * H + 7) / 8);
  return launch_core<true>(a, N > 32 ? 2 : 1, d > 32 ? 2 : 1, soft_reset != 0,
                           static_cast<hipStream_t>(stream));
}
