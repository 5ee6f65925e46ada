// Spike attention in the reference's linear order, for gfx950.
//
// snnk_spike_av_lif replaces spike_av_lif / _spike_av_lif_kernel
// (snn_compiler/kernels/attention.py:49-137): for each batch*head and step t,
// a = q_t @ kv_t, v = decay*v + in_scale*a, spike, reset.  The membrane stays
// in registers across T and `a` is never written to memory.
//
// linear_attention_kernel is the large-shape path of snnk_spike_attention
// (more than 64 tokens or more than 64 dims per head): per step the block
// forms KV_t = K_t^T V_t on MFMA from the K and V spikes, then the same
// q @ KV + LIF.  Over the integers Q (K^T V) == (Q K^T) V, so its counts
// equal those of the quadratic core in attention.hip.
//
// Both products run on v_mfma_f32_32x32x16_bf16 with fp32 accumulation,
// formed transposed (a^T = kv^T q^T) so that the accumulator of a lane holds
// four consecutive output dims of one token in each register quad: one
// vector store per 4 spikes.  kv enters the MFMA as P bf16 parts whose exact
// sum is its fp32 value (hi and mid keep 8 significant bits by truncation,
// lo the remaining at most 8), so every product of a 0/1 q with kv is exact
// and the fp32 accumulator holds the exact sum whenever it is an integer
// below 2^24.  P = 3 covers any fp32 kv; integer counts up to 256 need one
// part and up to 65535 two.
#include "snnk_common.h"

namespace snnk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format
constexpr uint32_t kFar = 0x80000000u;   // offset past every descriptor's range: reads 0
constexpr int kMaxThreads = 512;

// x == hi + mid + lo exactly, each a bf16 (returned as raw 16-bit patterns).
__device__ __forceinline__ void split_bf16(float x, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  const uint32_t h = __float_as_uint(x) & 0xFFFF0000u;
  const float r1 = __fsub_rn(x, __uint_as_float(h));  // the low 16 significand bits, exact
  const uint32_t m = __float_as_uint(r1) & 0xFFFF0000u;
  const float r2 = __fsub_rn(r1, __uint_as_float(m));  // at most 8 significant bits, exact
  hi = h >> 16;
  mid = m >> 16;
  lo = __float_as_uint(r2) >> 16;
}

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) { return lo | (hi << 16); }

// element types of q / the output spikes
template <int QT>
struct Elem {
  static constexpr int kBytes = QT == SNNK_F32 ? 4 : 2;
  static constexpr uint32_t kOne = QT == SNNK_F32 ? 0x3F800000u : (QT == SNNK_BF16 ? 0x3F80u : 0x3C00u);
  // one element (raw bits) -> bf16 bits
  __device__ static __forceinline__ uint32_t to_bf16(uint32_t raw) {
    if constexpr (QT == SNNK_F32) return f32_to_bf16_rne(__uint_as_float(raw));
    else if constexpr (QT == SNNK_BF16) return raw & 0xFFFFu;
    else return f32_to_bf16_rne(f16_to_f32(static_cast<uint16_t>(raw)));
  }
};

// 8 consecutive elements of a row (raw bits), from a buffer descriptor whose
// out-of-range offsets read zeros.  `vec`: the 8 elements are one aligned
// 16 / 32-byte run, read with vector loads; otherwise element by element,
// with element i valid when i < n_ok.
template <int QT>
__device__ __forceinline__ bf16x8 load_frag(__amdgpu_buffer_rsrc_t r, uint32_t off, bool vec, int n_ok) {
  uint32_t w[4];
  if (vec) {
    if constexpr (QT == SNNK_F32) {
      const i32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
      const i32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(r, off == kFar ? kFar : off + 16u, 0, 0);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        w[i] = pack2(Elem<QT>::to_bf16(static_cast<uint32_t>(lo[2 * i])),
                     Elem<QT>::to_bf16(static_cast<uint32_t>(lo[2 * i + 1])));
        w[2 + i] = pack2(Elem<QT>::to_bf16(static_cast<uint32_t>(hi[2 * i])),
                         Elem<QT>::to_bf16(static_cast<uint32_t>(hi[2 * i + 1])));
      }
    } else {
      const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t x = static_cast<uint32_t>(v[i]);
        w[i] = pack2(Elem<QT>::to_bf16(x & 0xFFFFu), Elem<QT>::to_bf16(x >> 16));
      }
    }
  } else {
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t o = (off == kFar || i >= n_ok) ? kFar : off + i * Elem<QT>::kBytes;
      uint32_t raw;
      if constexpr (QT == SNNK_F32) raw = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0));
      else raw = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, o, 0, 0));
      e[i] = Elem<QT>::to_bf16(raw);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack2(e[2 * i], e[2 * i + 1]);
  }
  bf16x8 f;
  __builtin_memcpy(&f, w, 16);
  return f;
}

// One LIF step on the 16 accumulator values of a lane; bit e of the result
// is the spike of register e.  Every product and sum is rounded to fp32 in
// the reference's order (decay*v + in_scale*a).
__device__ __forceinline__ uint32_t lif16(const f32x16& acc, float (&vm)[16], float decay,
                                          float in_scale, float vth, float v_reset, bool soft) {
  uint32_t bits = 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float h = __fadd_rn(__fmul_rn(decay, vm[e]), __fmul_rn(in_scale, acc[e]));
    const bool s = h >= vth;
    vm[e] = s ? (soft ? __fsub_rn(h, vth) : v_reset) : h;
    bits |= s ? (1u << e) : 0u;
  }
  return bits;
}

// ============================ snnk_spike_av_lif ==============================
struct AvArgs {
  const unsigned char* q;   // [T][BH][N][d] of the q type
  const unsigned char* kv;  // [T][BH][d][d] fp32 or int32
  unsigned char* out;       // [T][BH][N][d] of the q type
  int T, BH, N, d;
  int ntn;                  // 32-token tiles: ceil(N / 32)
  int nch;                  // token tiles per block (waves = nch * NTJ)
  int chunks;               // blocks per batch*head
  int ks;                   // 16-wide k steps: ceil(d / 16)
  int kgroups;              // 8-wide k groups: ceil(d / 8)
  int per_xcd;              // blocks per XCD
  float decay, in_scale, vth, v_reset;
  int soft_reset;
  int vec;                  // d % 8 == 0 and q / out 16-byte aligned
  int kv_int;               // kv holds int32
};

// Block = nch x NTJ waves for one batch*head and nch token tiles; wave w owns
// output tile (token tile ch*nch + w/NTJ, dim tile w%NTJ) for all T steps.
// Per step the block stages kv_t^T as three bf16 parts in LDS ([part][j][k],
// rows padded to 16 bytes past the k range: conflict-free fragment reads).
template <int NTJ, int QT>
__global__ __launch_bounds__(kMaxThreads) void spike_av_lif_kernel(AvArgs a) {
  constexpr int kJ = NTJ * 32;
  constexpr int kPitch = kJ + 8;
  constexpr int kPart = kJ * kPitch;
  constexpr int kE = Elem<QT>::kBytes;
  __shared__ __attribute__((aligned(16))) uint16_t kvs[3 * kPart];

  const int tid = threadIdx.x, nthreads = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, g = lane >> 5;
  // blocks are dealt to the 8 XCDs round-robin by id; each XCD takes a
  // contiguous range of (batch*head, chunk)
  const int blk = (blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (blk >= a.BH * a.chunks) return;  // whole block
  const int bh = blk / a.chunks, ch = blk - bh * a.chunks;
  const int nt = ch * a.nch + wave / NTJ, jt = wave % NTJ;
  const bool tile_ok = nt < a.ntn;      // wave-uniform
  const int n = nt * 32 + r32;          // this lane's token
  const bool n_ok = n < a.N;

  // padding rows (j >= d) and columns (k >= d) stay zero for the whole kernel
  for (int i = tid; i < 3 * kPart / 8; i += nthreads)
    reinterpret_cast<u32x4*>(kvs)[i] = u32x4{0u, 0u, 0u, 0u};

  float vm[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) vm[e] = 0.0f;
  const int64_t q_slice = static_cast<int64_t>(a.N) * a.d;   // elements per (t, bh)
  const int64_t kv_slice = static_cast<int64_t>(a.d) * a.d;
  const bool soft = a.soft_reset != 0;

  for (int t = 0; t < a.T; ++t) {
    const int64_t sl = static_cast<int64_t>(t) * a.BH + bh;
    // ---- this lane's q fragments (B operand: token n, dims 16kk + 8g ..) ----
    bf16x8 fq[2 * NTJ];
    {
      const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<unsigned char*>(a.q + sl * q_slice * kE), 0,
          static_cast<int>(q_slice * kE), kRsrcWord3);
#pragma unroll
      for (int kk = 0; kk < 2 * NTJ; ++kk) {
        const int k0 = kk * 16 + 8 * g;
        const uint32_t off = (tile_ok && n_ok && kk < a.ks && k0 < a.d)
                                 ? static_cast<uint32_t>((n * a.d + k0) * kE) : kFar;
        fq[kk] = load_frag<QT>(qr, off, a.vec != 0, a.d - k0);
      }
    }
    // ---- stage kv_t^T: item (j, k group): 8 strided loads, 3 LDS rows -------
    __syncthreads();  // the previous step's fragment reads are done
    {
      const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<unsigned char*>(a.kv + sl * kv_slice * 4), 0,
          static_cast<int>(kv_slice * 4), kRsrcWord3);
      const int n_items = a.d * a.kgroups;
      for (int it = tid; it < n_items; it += nthreads) {
        const int kgi = it / a.d, j = it - kgi * a.d;
        uint32_t part[3][4];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int k = kgi * 8 + i;
          const uint32_t off = k < a.d ? static_cast<uint32_t>((k * a.d + j) * 4) : kFar;
          const uint32_t raw = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(kr, off, 0, 0));
          const float x = a.kv_int ? static_cast<float>(static_cast<int32_t>(raw)) : __uint_as_float(raw);
          uint32_t h, m, l;
          split_bf16(x, h, m, l);
          const int sh = (i & 1) * 16;
          if ((i & 1) == 0) { part[0][i / 2] = h; part[1][i / 2] = m; part[2][i / 2] = l; }
          else { part[0][i / 2] |= h << sh; part[1][i / 2] |= m << sh; part[2][i / 2] |= l << sh; }
        }
#pragma unroll
        for (int p = 0; p < 3; ++p)
          *reinterpret_cast<u32x4*>(kvs + p * kPart + j * kPitch + kgi * 8) =
              u32x4{part[p][0], part[p][1], part[p][2], part[p][3]};
      }
    }
    __syncthreads();
    if (!tile_ok) continue;  // wave-uniform; the wave still meets every barrier

    // ---- a^T tile = kv^T q^T, exact parts -----------------------------------
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
    const uint16_t* arow = kvs + (jt * 32 + r32) * kPitch + 8 * g;
#pragma unroll
    for (int kk = 0; kk < 2 * NTJ; ++kk) {
      if (kk < a.ks) {
        const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(arow + kk * 16);
        const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(arow + kPart + kk * 16);
        const bf16x8 a2 = *reinterpret_cast<const bf16x8*>(arow + 2 * kPart + kk * 16);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, fq[kk], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, fq[kk], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, fq[kk], acc, 0, 0, 0);
      }
    }
    // ---- LIF and the spikes of token n, dims jt*32 + 8*e4 + 4*g + 0..3 ------
    const uint32_t bits = lif16(acc, vm, a.decay, a.in_scale, a.vth, a.v_reset, soft);
    if (n_ok) {
      unsigned char* orow = a.out + (sl * q_slice + static_cast<int64_t>(n) * a.d) * kE;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int j0 = jt * 32 + 8 * e4 + 4 * g;
        if (j0 >= a.d) continue;
        uint32_t s[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) s[x] = ((bits >> (4 * e4 + x)) & 1u) ? Elem<QT>::kOne : 0u;
        if (a.vec) {
          if constexpr (kE == 4) *reinterpret_cast<u32x4*>(orow + j0 * 4) = u32x4{s[0], s[1], s[2], s[3]};
          else *reinterpret_cast<u32x2*>(orow + j0 * 2) = u32x2{pack2(s[0], s[1]), pack2(s[2], s[3])};
        } else {
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            if (j0 + x >= a.d) break;
            if constexpr (kE == 4) reinterpret_cast<uint32_t*>(orow)[j0 + x] = s[x];
            else reinterpret_cast<uint16_t*>(orow)[j0 + x] = static_cast<uint16_t>(s[x]);
          }
        }
      }
    }
  }
}

// ===================== snnk_spike_attention, large shapes =====================
struct LinArgs {
  const uint16_t* q;  // bf16 spikes, element (t, b*N + n, h*d + dd)
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_row, k_row, v_row;  // row strides (elements)
  int64_t q_t, k_t, v_t;        // step strides (elements)
  uint16_t* out;                // bf16 spikes (t, b*N + n, h*d + dd)
  int64_t o_row, o_t;
  int32_t* o_counts;            // optional [T][B][H][N][d]
  int T, B, H, N, d;
  int ntn, nch, chunks, per_xcd;
  int ks;                       // ceil(d / 16)
  int kgroups;                  // d / 8
  int tok_chunks;               // ceil(N / 64)
  float decay, in_scale, vth, v_reset;
  int soft_reset;
  int o_vec;                    // output rows and steps 8-byte aligned
};

constexpr int kTok = 64;  // tokens of K and V staged per chunk

// Block = nch x NTJ waves for one (batch, head) and nch token tiles.  Per step:
//  1. K_t^T and V_t^T in 64-token chunks into LDS (bf16, [dim][token]); the
//     waves take the NTJ x NTJ tiles of KV_t = K_t^T V_t round-robin and
//     accumulate them over the chunks (exact counts <= N in fp32);
//  2. KV_t^T as P bf16 parts into LDS ([part][j][k]);
//  3. as in spike_av_lif_kernel: a^T = KV^T q^T per wave tile, LIF, spikes.
template <int NTJ, int P>
__global__ __launch_bounds__(kMaxThreads) void linear_attention_kernel(LinArgs a) {
  constexpr int kJ = NTJ * 32;
  constexpr int kSPitch = kTok + 8;  // bf16 per staged [dim] row
  constexpr int kPitch = kJ + 8;
  constexpr int kPart = kJ * kPitch;
  constexpr int kMaxKvTiles = NTJ;   // KV tiles per wave: NTJ^2 tiles over >= NTJ waves
  __shared__ __attribute__((aligned(16))) uint16_t kts[kJ * kSPitch];
  __shared__ __attribute__((aligned(16))) uint16_t vts[kJ * kSPitch];
  __shared__ __attribute__((aligned(16))) uint16_t kvs[P * kPart];

  const int tid = threadIdx.x, nthreads = blockDim.x;
  const int nwaves = nthreads >> 6;
  const int lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, g = lane >> 5;
  const int blk = (blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (blk >= a.B * a.H * a.chunks) return;  // whole block
  const int bh = blk / a.chunks, ch = blk - bh * a.chunks;
  const int b = bh / a.H, h = bh - b * a.H;
  const int nt = ch * a.nch + wave / NTJ, jt = wave % NTJ;
  const bool tile_ok = nt < a.ntn;
  const int n = nt * 32 + r32;
  const bool n_ok = n < a.N;
  const int64_t row0 = static_cast<int64_t>(b) * a.N;
  const uint16_t* qb = a.q + row0 * a.q_row + h * a.d;
  const uint16_t* kb = a.k + row0 * a.k_row + h * a.d;
  const uint16_t* vb = a.v + row0 * a.v_row + h * a.d;
  constexpr int kRecords = 0x7FFFFFFF;

  // staged rows of dims >= d stay zero for the whole kernel
  for (int i = tid; i < kJ * kSPitch / 8; i += nthreads) {
    reinterpret_cast<u32x4*>(kts)[i] = u32x4{0u, 0u, 0u, 0u};
    reinterpret_cast<u32x4*>(vts)[i] = u32x4{0u, 0u, 0u, 0u};
  }

  float vm[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) vm[e] = 0.0f;
  const bool soft = a.soft_reset != 0;
  const int n_kv_tiles = NTJ * NTJ;
  // staging items per tensor: (8-dim group, token pair) of one 64-token chunk
  const int n_items = a.kgroups * (kTok / 2);

  for (int t = 0; t < a.T; ++t) {
    // q fragments of this lane (B operand), in flight during the KV phase
    bf16x8 fq[2 * NTJ];
    {
      const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(qb + t * a.q_t), 0, kRecords, kRsrcWord3);
#pragma unroll
      for (int kk = 0; kk < 2 * NTJ; ++kk) {
        const int k0 = kk * 16 + 8 * g;
        const uint32_t off = (tile_ok && n_ok && k0 < a.d)
                                 ? static_cast<uint32_t>((n * a.q_row + k0) * 2) : kFar;
        const i32x4 v4 = __builtin_amdgcn_raw_buffer_load_b128(qr, off, 0, 0);
        __builtin_memcpy(&fq[kk], &v4, 16);
      }
    }
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(kb + t * a.k_t), 0, kRecords, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(vb + t * a.v_t), 0, kRecords, kRsrcWord3);

    f32x16 kacc[kMaxKvTiles];
#pragma unroll
    for (int m = 0; m < kMaxKvTiles; ++m)
#pragma unroll
      for (int e = 0; e < 16; ++e) kacc[m][e] = 0.0f;

    for (int c = 0; c < a.tok_chunks; ++c) {
      // ---- stage the chunk: item (dim group dg, token pair tp) ------------------
      for (int it = tid; it < n_items; it += nthreads) {
        const int dg = it >> 5, tp = it & 31;
        const int n0 = c * kTok + 2 * tp;
        const uint32_t ok0 = n0 < a.N, ok1 = n0 + 1 < a.N;
        const uint32_t k0o = ok0 ? static_cast<uint32_t>((n0 * a.k_row + dg * 8) * 2) : kFar;
        const uint32_t k1o = ok1 ? static_cast<uint32_t>(((n0 + 1) * a.k_row + dg * 8) * 2) : kFar;
        const uint32_t v0o = ok0 ? static_cast<uint32_t>((n0 * a.v_row + dg * 8) * 2) : kFar;
        const uint32_t v1o = ok1 ? static_cast<uint32_t>(((n0 + 1) * a.v_row + dg * 8) * 2) : kFar;
        const i32x4 k0 = __builtin_amdgcn_raw_buffer_load_b128(kr, k0o, 0, 0);
        const i32x4 k1 = __builtin_amdgcn_raw_buffer_load_b128(kr, k1o, 0, 0);
        const i32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(vr, v0o, 0, 0);
        const i32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(vr, v1o, 0, 0);
        // dims 2p, 2p+1 of tokens n0, n0+1 -> LDS words (n0, n0+1) of rows 2p, 2p+1
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const int r = dg * 8 + 2 * p;
          uint32_t* kt0 = reinterpret_cast<uint32_t*>(kts + r * kSPitch + 2 * tp);
          uint32_t* vt0 = reinterpret_cast<uint32_t*>(vts + r * kSPitch + 2 * tp);
          kt0[0] = __builtin_amdgcn_perm(static_cast<uint32_t>(k1[p]), static_cast<uint32_t>(k0[p]), 0x05040100u);
          kt0[kSPitch / 2] = __builtin_amdgcn_perm(static_cast<uint32_t>(k1[p]), static_cast<uint32_t>(k0[p]), 0x07060302u);
          vt0[0] = __builtin_amdgcn_perm(static_cast<uint32_t>(v1[p]), static_cast<uint32_t>(v0[p]), 0x05040100u);
          vt0[kSPitch / 2] = __builtin_amdgcn_perm(static_cast<uint32_t>(v1[p]), static_cast<uint32_t>(v0[p]), 0x07060302u);
        }
      }
      __syncthreads();
      // ---- KV tiles: D[k][j] = sum_n K^T[k][n] V^T[j][n] -----------------------
#pragma unroll
      for (int m = 0; m < kMaxKvTiles; ++m) {
        const int tile = wave + m * nwaves;
        if (tile < n_kv_tiles) {
          const int kt = tile / NTJ, jt2 = tile - kt * NTJ;
          const uint16_t* ar = kts + (kt * 32 + r32) * kSPitch + 8 * g;
          const uint16_t* br = vts + (jt2 * 32 + r32) * kSPitch + 8 * g;
#pragma unroll
          for (int kk = 0; kk < kTok / 16; ++kk)
            kacc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                *reinterpret_cast<const bf16x8*>(ar + kk * 16),
                *reinterpret_cast<const bf16x8*>(br + kk * 16), kacc[m], 0, 0, 0);
        }
      }
      __syncthreads();  // the chunk's LDS reads are done before the next staging
    }
    // ---- KV^T parts: lane holds column j of KV, rows k = kt*32 + 8*e4 + 4*g + x
#pragma unroll
    for (int m = 0; m < kMaxKvTiles; ++m) {
      const int tile = wave + m * nwaves;
      if (tile < n_kv_tiles) {
        const int kt = tile / NTJ, jt2 = tile - kt * NTJ;
        const int j = jt2 * 32 + r32;
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          uint32_t ph[3][4];
#pragma unroll
          for (int x = 0; x < 4; ++x) split_bf16(kacc[m][4 * e4 + x], ph[0][x], ph[1][x], ph[2][x]);
          const int k0 = kt * 32 + 8 * e4 + 4 * g;
#pragma unroll
          for (int p = 0; p < P; ++p)
            *reinterpret_cast<u32x2*>(kvs + p * kPart + j * kPitch + k0) =
                u32x2{pack2(ph[p][0], ph[p][1]), pack2(ph[p][2], ph[p][3])};
        }
      }
    }
    __syncthreads();
    if (!tile_ok) continue;  // wave-uniform; the wave still meets every barrier

    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
    const uint16_t* arow = kvs + (jt * 32 + r32) * kPitch + 8 * g;
#pragma unroll
    for (int kk = 0; kk < 2 * NTJ; ++kk) {
      if (kk < a.ks) {
#pragma unroll
        for (int p = 0; p < P; ++p)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              *reinterpret_cast<const bf16x8*>(arow + p * kPart + kk * 16), fq[kk], acc, 0, 0, 0);
      }
    }
    if (a.o_counts && n_ok) {
      int32_t* oc = a.o_counts + ((static_cast<int64_t>(t) * a.B * a.H + bh) * a.N + n) * a.d;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int dd = jt * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
        if (dd < a.d) oc[dd] = static_cast<int32_t>(acc[e]);
      }
    }
    const uint32_t bits = lif16(acc, vm, a.decay, a.in_scale, a.vth, a.v_reset, soft);
    if (n_ok) {
      uint16_t* ot = a.out + t * a.o_t + (row0 + n) * a.o_row + h * a.d;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int j0 = jt * 32 + 8 * e4 + 4 * g;
        if (j0 >= a.d) continue;  // d % 8 == 0: all four dims are in range
        uint32_t s[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) s[x] = ((bits >> (4 * e4 + x)) & 1u) ? 0x3F80u : 0u;
        if (a.o_vec) {
          *reinterpret_cast<u32x2*>(ot + j0) = u32x2{pack2(s[0], s[1]), pack2(s[2], s[3])};
        } else {
#pragma unroll
          for (int x = 0; x < 4; ++x) ot[j0 + x] = static_cast<uint16_t>(s[x]);
        }
      }
    }
  }
}

// token tiles per block and blocks per batch*head: at most 8 waves, and
// blocks split further while the grid has fewer than `target` blocks
void plan_chunks(int ntn, int ntj, int64_t bh, int target, int* nch, int* chunks) {
  int c = std::max(1, std::min(8 / ntj, ntn));
  while (c > 1 && bh * ((ntn + c - 1) / c) < target) --c;
  *nch = c;
  *chunks = (ntn + c - 1) / c;
}

template <int QT>
int launch_av(const AvArgs& a, int ntj, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.per_xcd) * 8u), block(64 * a.nch * ntj);
  switch (ntj) {
    case 1: hipLaunchKernelGGL((spike_av_lif_kernel<1, QT>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((spike_av_lif_kernel<2, QT>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((spike_av_lif_kernel<3, QT>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((spike_av_lif_kernel<4, QT>), grid, block, 0, s, a); break;
    default: return SNNK_EUNSUPPORTED;
  }
  return launch_status();
}

template <int NTJ>
void launch_linear(const LinArgs& a, int parts, dim3 grid, dim3 block, hipStream_t s) {
  if (parts == 1) hipLaunchKernelGGL((linear_attention_kernel<NTJ, 1>), grid, block, 0, s, a);
  else if (parts == 2) hipLaunchKernelGGL((linear_attention_kernel<NTJ, 2>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((linear_attention_kernel<NTJ, 3>), grid, block, 0, s, a);
}

}  // namespace

// Large-shape path of snnk_spike_attention (called from attention.hip after
// its own argument checks): N > 64 or d > 64, d <= 128, d % 8 == 0, no S counts.
int spike_attention_linear(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           int64_t q_row, int64_t k_row, int64_t v_row, int64_t q_step,
                           int64_t k_step, int64_t v_step, uint16_t* spikes_out,
                           int64_t out_row, int64_t out_step, int32_t* o_counts, int64_t T,
                           int64_t B, int64_t H, int64_t N, int64_t d, float decay,
                           float in_scale, float v_threshold, float v_reset, int32_t soft_reset,
                           hipStream_t s) {
  if (d > 128 || d % 8 != 0) return SNNK_EUNSUPPORTED;
  // exact counts: a = q . KV <= d * N must stay below 2^24
  if (d * N >= (int64_t{1} << 24)) return SNNK_EUNSUPPORTED;
  // byte offsets of a (t, b, h) slice's rows are 32-bit
  const int64_t max_row = std::max(q_row, std::max(k_row, v_row));
  if ((N + 1) * max_row * 2 >= (int64_t{1} << 31)) return SNNK_EUNSUPPORTED;
  LinArgs a{};
  a.q = q; a.k = k; a.v = v;
  a.q_row = q_row; a.k_row = k_row; a.v_row = v_row;
  a.q_t = q_step; a.k_t = k_step; a.v_t = v_step;
  a.out = spikes_out; a.o_row = out_row; a.o_t = out_step;
  a.o_counts = o_counts;
  a.T = static_cast<int>(T); a.B = static_cast<int>(B); a.H = static_cast<int>(H);
  a.N = static_cast<int>(N); a.d = static_cast<int>(d);
  const int ntj = static_cast<int>((d + 31) / 32);
  a.ntn = static_cast<int>((N + 31) / 32);
  plan_chunks(a.ntn, ntj, B * H, 256, &a.nch, &a.chunks);
  const int64_t blocks = B * H * a.chunks;
  if (blocks > 0x7FFFFFF0ll) return SNNK_EUNSUPPORTED;
  a.per_xcd = static_cast<int>((blocks + 7) / 8);
  a.ks = static_cast<int>((d + 15) / 16);
  a.kgroups = static_cast<int>(d / 8);
  a.tok_chunks = static_cast<int>((N + kTok - 1) / kTok);
  a.decay = decay; a.in_scale = in_scale; a.vth = v_threshold; a.v_reset = v_reset;
  a.soft_reset = soft_reset ? 1 : 0;
  a.o_vec = aligned(spikes_out, 8) && out_row % 4 == 0 && out_step % 4 == 0;
  // one bf16 part for counts up to 256, two below 65536
  const int parts = N <= 256 ? 1 : (N < 65536 ? 2 : 3);
  const dim3 grid(static_cast<unsigned>(a.per_xcd) * 8u), block(64 * a.nch * ntj);
  switch (ntj) {
    case 1: launch_linear<1>(a, parts, grid, block, s); break;
    case 2: launch_linear<2>(a, parts, grid, block, s); break;
    case 3: launch_linear<3>(a, parts, grid, block, s); break;
    default: launch_linear<4>(a, parts, grid, block, s); break;
  }
  return launch_status();
}

}  // namespace snnk

using namespace snnk;

extern "C" int snnk_spike_av_lif(const void* q, int32_t q_dtype, const void* kv, int32_t kv_dtype,
                                 void* spikes_out, int64_t T, int64_t BH, int64_t N, int64_t d,
                                 float decay, float in_scale, float v_threshold, float v_reset,
                                 int32_t soft_reset, void* stream) {
  if (T < 0 || BH < 0 || N < 0 || d <= 0) return SNNK_EINVAL;
  if (T == 0 || BH == 0 || N == 0) return SNNK_OK;
  if (q == nullptr || kv == nullptr || spikes_out == nullptr) return SNNK_EINVAL;
  if (q_dtype != SNNK_F32 && q_dtype != SNNK_BF16 && q_dtype != SNNK_F16) return SNNK_EINVAL;
  if (kv_dtype != SNNK_F32 && kv_dtype != SNNK_I32) return SNNK_EINVAL;
  if (d > 128) return SNNK_EUNSUPPORTED;
  const int esize = q_dtype == SNNK_F32 ? 4 : 2;
  // one (t, batch*head) slice of q and of kv is addressed with 31-bit byte offsets
  if (N * d * esize >= (int64_t{1} << 31) || T * BH >= (int64_t{1} << 31))
    return SNNK_EUNSUPPORTED;
  if (!aligned(q, esize) || !aligned(kv, 4) || !aligned(spikes_out, esize)) return SNNK_EALIGN;
  AvArgs a{};
  a.q = static_cast<const unsigned char*>(q);
  a.kv = static_cast<const unsigned char*>(kv);
  a.out = static_cast<unsigned char*>(spikes_out);
  a.T = static_cast<int>(T); a.BH = static_cast<int>(BH);
  a.N = static_cast<int>(N); a.d = static_cast<int>(d);
  const int ntj = static_cast<int>((d + 31) / 32);
  a.ntn = static_cast<int>((N + 31) / 32);
  plan_chunks(a.ntn, ntj, BH, 512, &a.nch, &a.chunks);
  const int64_t blocks = BH * a.chunks;
  if (blocks > 0x7FFFFFF0ll) return SNNK_EUNSUPPORTED;
  a.per_xcd = static_cast<int>((blocks + 7) / 8);
  a.ks = static_cast<int>((d + 15) / 16);
  a.kgroups = static_cast<int>((d + 7) / 8);
  a.decay = decay; a.in_scale = in_scale; a.vth = v_threshold; a.v_reset = v_reset;
  a.soft_reset = soft_reset ? 1 : 0;
  a.vec = d % 8 == 0 && aligned(q, 16) && aligned(spikes_out, 16);
  a.kv_int = kv_dtype == SNNK_I32;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (q_dtype) {
    case SNNK_F32: return launch_av<SNNK_F32>(a, ntj, s);
    case SNNK_BF16: return launch_av<SNNK_BF16>(a, ntj, s);
    default: return launch_av<SNNK_F16>(a, ntj, s);
  }
}
