// Bit-packed binary GEMM on int8 MFMA (gfx950 v_mfma_i32_32x32x32_i8).
//
//   C[b][m][n] = sum_k A01[m][k] * B01[n][k]                (unsigned)
//   C[b][m][n] = 2 * sum_k A01*B01 - sum_k A01[m][k]         (signed weights)
// with A, B packed along k as uint32 words (bit k%32 of word k/32).
//
// Each wave owns a (32*TM)x(32*TN) tile of C as TMxTN MFMA 32x32 accumulators
// and walks K in stages of 4 words (128 bits) staged through an LDS ring.
// With TM x TN = 2 x 4 two waves fit a SIMD, so one wave's result stores
// overlap the other's MFMAs.  A packed 32-bit word feeds one MFMA
// k-step (32 int8 k values): the lane half g (lane/32) builds its 16 operand
// bytes as the 4 dwords (w >> (4g+s)) & 0x01010101, s = 0..3, i.e. byte b of
// dword s holds bit 4g+s+8b.  A and B operands use this same bit->k
// assignment, so every bit of A meets the matching bit of B in the
// contraction whatever the instruction's internal k order is.
//
// A second kernel runs the same tiling on the gfx950 MX-scaled fp4 MFMA
// (v_mfma_scale_f32_32x32x64_f8f6f4, e2m1 operands, block scales 2^0): a bit
// becomes an e2m1 nibble that is 0 or a power of two, chosen so that every
// product of two set bits is exactly 1 (A and B carry reciprocal values at
// each nibble position); the fp32 accumulator holds the exact count (at most
// K < 2^24).  A 32-bit word feeds one lane's 32 k values of a k-step of 64
// (lane half g takes word g of the pair): nibble j of dword s holds bit 4j+s,
// for A and B alike.  Per k, this is half the MFMA time and under half the
// unpacking work of the int8 kernel.
#include "snnk_common.h"

namespace snnk {

int popcount_gemm(const uint32_t* A, const uint32_t* B, void* C, int32_t c_dtype,
                  int64_t batch, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                  int64_t ldc, int64_t sA, int64_t sB, int64_t sC, int signed_w,
                  hipStream_t s);

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kStageW = 4;     // packed words per stage

typedef __attribute__((address_space(3))) void* lds_ptr_t;
constexpr uint32_t kOOB = 0xFFFFFFF0u;        // buffer offset past every operand
constexpr int kRsrcWord3 = 0x00020000;       // raw buffer, 32-bit data format
// Stages in the LDS ring: 8 for a 128x128 wave tile (32 KB); 6 for the
// 128x64 tile (18 KB), so that eight such waves -- two per SIMD -- fit a CU.
template <int TM, int TN>
constexpr int ring_depth() { return TM * TN >= 16 ? 8 : 6; }
template <int TM, int TN>
constexpr int waves_per_simd() { return TM * TN >= 16 ? 1 : 2; }

__device__ __forceinline__ i32x4 expand(uint32_t w, int g) {
  const uint32_t x = w >> (4 * g);
  i32x4 r;
  r[0] = static_cast<int>(x & 0x01010101u);
  r[1] = static_cast<int>((x >> 1) & 0x01010101u);
  r[2] = static_cast<int>((x >> 2) & 0x01010101u);
  r[3] = static_cast<int>((x >> 3) & 0x01010101u);
  return r;
}

// 4 MFMA k-steps of one stage for the wave's TM x TN accumulator tiles.
template <bool SIGNED, int TM, int TN>
__device__ __forceinline__ void mfma_stage(i32x16 (&acc)[TM][TN], const u32x4 (&a)[TM],
                                           const u32x4 (&b)[TN], int g, int (&rowpop)[TM]) {
#pragma unroll
  for (int kk = 0; kk < kStageW; ++kk) {
    i32x4 fa[TM], fb[TN];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      fa[t] = expand(a[t][kk], g);
      if constexpr (SIGNED) rowpop[t] += __builtin_popcount(a[t][kk]);
    }
#pragma unroll
    for (int t = 0; t < TN; ++t) fb[t] = expand(b[t][kk], g);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
  }
}

// Largest row pitch (elements) of C for which every offset inside a
// 128-row tile fits the 32-bit buffer offsets of store_tile's fast path.
constexpr int64_t kMaxFastLdc = int64_t{1} << 22;

// Writes a wave's TM x TN tiles of 32x32 counts (SIGNED: 2*count - rowpop).
// Accumulator register e of lane l holds row 8*(e/4) + 4*(l/32) + e%4,
// column l%32 of its tile.  A wave tile wholly inside C (every tile of a
// shape that the tiles divide) is written by buffer stores whose row offset
// is wave-uniform (an SGPR) and whose column offset is an immediate: no
// per-element bounds branch and no 64-bit address arithmetic (3.5 KB of code
// for a 128x128 fp4 tile against 17 KB for the checked path, which every
// launch would fetch from a cold instruction cache).
template <bool SIGNED, bool OUT_F32, int TM, int TN, typename Acc>
__device__ __forceinline__ void store_tile(const Acc (&acc)[TM][TN], const int (&rowpop)[TM],
                                           void* Cb, int64_t M, int64_t N, int64_t ldc,
                                           int64_t m_base, int64_t n_base, int lane) {
  const int r32 = lane & 31, g = lane >> 5;
  auto value = [&](int i, int j, int e, int rp) __attribute__((always_inline)) {
    int32_t c = static_cast<int32_t>(acc[i][j][e]);  // exact integer count
    if constexpr (SIGNED) c = 2 * c - rp;
    if constexpr (OUT_F32) return __float_as_uint(static_cast<float>(c));
    else return static_cast<uint32_t>(c);
  };
  if (m_base + 32 * TM <= M && n_base + 32 * TN <= N && ldc <= kMaxFastLdc) {
    uint32_t* base = static_cast<uint32_t*>(Cb) + m_base * ldc + n_base;
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(base, 0, -1, kRsrcWord3);
    const uint32_t ldc4 = static_cast<uint32_t>(ldc) * 4u;
    const uint32_t voff = static_cast<uint32_t>(4 * g) * ldc4 + static_cast<uint32_t>(r32) * 4u;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        int rp = 0;
        if constexpr (SIGNED) rp = __shfl(rowpop[i], 8 * (e >> 2) + 4 * g + (e & 3), 64);
        const uint32_t soff = static_cast<uint32_t>(i * 32 + 8 * (e >> 2) + (e & 3)) * ldc4;
#pragma unroll
        for (int j = 0; j < TN; ++j)  // non-temporal (aux bit 1): the counts are not re-read here
          __builtin_amdgcn_raw_buffer_store_b32(value(i, j, e, rp), rc, voff + j * 128, soff, 2);
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int rr = 8 * (e >> 2) + 4 * g + (e & 3);
      int rp = 0;
      if constexpr (SIGNED) rp = __shfl(rowpop[i], rr, 64);
      const int64_t m = m_base + i * 32 + rr;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t n = n_base + j * 32 + r32;
        if (m < M && n < N)
          __builtin_nontemporal_store(value(i, j, e, rp), static_cast<uint32_t*>(Cb) + m * ldc + n);
      }
    }
  }
}

// One wave per workgroup.  The packed words of each stage (4 per row: 16
// bytes for each of the 32*TM A rows and 32*TN B rows) arrive by direct
// global->LDS buffer loads into a kRing-deep ring, kRing-1 stages ahead, so
// no barrier is needed (one wave) and the load latency stays hidden.  Rows
// past M / N read as zeros (range-checked offsets); in the last stage words
// past KW are cleared and the bits past K of the last word masked.
template <bool SIGNED, bool OUT_F32, int TM, int TN>
__global__ __launch_bounds__(64)
__attribute__((amdgpu_waves_per_eu(waves_per_simd<TM, TN>()))) void bgemm_mfma_kernel(
    const uint32_t* __restrict__ A, const uint32_t* __restrict__ B, void* __restrict__ Cv,
    int64_t M, int64_t N, int64_t KW, uint32_t last_mask, int64_t lda, int64_t ldb,
    int64_t ldc, int64_t sA, int64_t sB, int64_t sC, uint32_t a_bytes, uint32_t b_bytes) {
  constexpr int kRows = 32 * (TM + TN);          // rows per stage, A then B
  constexpr int kRing = ring_depth<TM, TN>();
  __shared__ __attribute__((aligned(1024))) u32x4 ring[kRing][kRows];
  const int lane = threadIdx.x;
  const int r32 = lane & 31, g = lane >> 5;
  const int64_t bz = blockIdx.z;
  const int64_t m_base = static_cast<int64_t>(blockIdx.y) * (32 * TM);
  const int64_t n_base = static_cast<int64_t>(blockIdx.x) * (32 * TN);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(A + bz * sA), 0, a_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(B + bz * sB), 0, b_bytes, kRsrcWord3);

  // lane l loads row 64*q + l of the stage (q-th 64-row group)
  constexpr int kGroups = kRows / 64;
  uint32_t row_off[kGroups];
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    const int r = 64 * q + lane;
    if (r < 32 * TM) {
      const int64_t m = m_base + r;
      row_off[q] = m < M ? static_cast<uint32_t>(m * lda * 4) : kOOB;
    } else {
      const int64_t n = n_base + (r - 32 * TM);
      row_off[q] = n < N ? static_cast<uint32_t>(n * ldb * 4) : kOOB;
    }
  }
  const int64_t n_stages = (KW + kStageW - 1) / kStageW;
  auto issue = [&](int64_t st, int buf) {
    const bool live = st < n_stages;
    const uint32_t d = static_cast<uint32_t>(st * kStageW * 4);
#pragma unroll
    for (int q = 0; q < kGroups; ++q) {
      const bool is_a = 64 * q < 32 * TM;  // compile-time after unrolling
      const uint32_t off = (live && row_off[q] != kOOB) ? row_off[q] + d : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? ra : rb, (lds_ptr_t)&ring[buf][64 * q], 16,
                                               off, 0, 0, 0);
    }
  };

  i32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;
  int rowpop[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) rowpop[t] = 0;

  // operands of stage st from its ring slot; the last stage clears words past
  // KW and masks the bits past K (uniform branch)
  auto read_stage = [&](u32x4 (&a)[TM], u32x4 (&b)[TN], int64_t st) {
    const int rb_ = static_cast<int>(st % kRing);
#pragma unroll
    for (int t = 0; t < TM; ++t) a[t] = ring[rb_][t * 32 + r32];
#pragma unroll
    for (int t = 0; t < TN; ++t) b[t] = ring[rb_][32 * TM + t * 32 + r32];
    if (st == n_stages - 1) {
      const int64_t w0 = st * kStageW;
#pragma unroll
      for (int j = 0; j < kStageW; ++j) {
        const uint32_t keep = w0 + j < KW - 1 ? 0xFFFFFFFFu : (w0 + j == KW - 1 ? last_mask : 0u);
#pragma unroll
        for (int t = 0; t < TM; ++t) a[t][j] &= keep;
#pragma unroll
        for (int t = 0; t < TN; ++t) b[t][j] &= keep;
      }
    }
  };

#pragma unroll
  for (int p = 0; p < kRing - 1; ++p) issue(p, p);
  for (int64_t s = 0; s < n_stages; ++s) {
    // stage s has landed once at most the kRing-2 stages after it are
    // outstanding (each stage is kGroups loads per lane)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kGroups * (kRing - 2)) : "memory");
    u32x4 a[TM], b[TN];
    read_stage(a, b, s);
    // refill the slot of stage s-1: its reads completed before last stage's
    // MFMAs consumed them (one wave per block, so no barrier)
    issue(s + kRing - 1, static_cast<int>((s + kRing - 1) % kRing));
    mfma_stage<SIGNED, TM, TN>(acc, a, b, g, rowpop);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing zero-fill loads

  // C elements are 4 bytes (int32 or fp32) either way
  store_tile<SIGNED, OUT_F32, TM, TN>(acc, rowpop, static_cast<uint32_t*>(Cv) + bz * sC, M, N, ldc,
                                      m_base, n_base, lane);
}

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// e2m1 operands of one lane for one k-step.  Nibble j of dword s carries
// bit 4j+s of the word w, as 0 or a power of two; the A and B values at each
// position are reciprocal, so every product of two set bits is exactly 1:
//   position s      0    1    2    3
//   B (5 ops)      0.5  1.0  2.0  1.0     (s = 0..2 keep their bit in place)
//   A (6 ops)      2.0  1.0  0.5  1.0
// (e2m1 nibbles: 0.5 = 0001 (subnormal), 1.0 = 0010, 2.0 = 0100.)
__device__ __forceinline__ i32x8 expand_f4_b(uint32_t w) {
  i32x8 r;
  r[0] = static_cast<int>(w & 0x11111111u);
  r[1] = static_cast<int>(w & 0x22222222u);
  r[2] = static_cast<int>(w & 0x44444444u);
  r[3] = static_cast<int>((w >> 2) & 0x22222222u);
  r[4] = r[5] = r[6] = r[7] = 0;  // fp4 operands use the first four dwords
  return r;
}
__device__ __forceinline__ i32x8 expand_f4_a(uint32_t w) {
  const uint32_t h = w >> 2;
  i32x8 r;
  r[0] = static_cast<int>((w << 2) & 0x44444444u);
  r[1] = static_cast<int>(w & 0x22222222u);
  r[2] = static_cast<int>(h & 0x11111111u);
  r[3] = static_cast<int>(h & 0x22222222u);
  r[4] = r[5] = r[6] = r[7] = 0;
  return r;
}

// Same tiling, ring and loads as bgemm_mfma_kernel; each lane reads the two
// words of its row that its half g consumes (g and g+2 of the 4-word stage)
// and a stage is two fp4 k-steps of 64.  Software pipelined: the LDS words
// of stage s+1 are read while stage s's MFMAs run, and the e2m1 operands of
// the next k-step are unpacked between the current k-step's MFMAs.
template <bool SIGNED, bool OUT_F32, int TM, int TN>
__global__ __launch_bounds__(64)
__attribute__((amdgpu_waves_per_eu(waves_per_simd<TM, TN>()))) void bgemm_f4_kernel(
    const uint32_t* __restrict__ A, const uint32_t* __restrict__ B, void* __restrict__ Cv,
    int64_t M, int64_t N, int64_t KW, uint32_t last_mask, int64_t lda, int64_t ldb,
    int64_t ldc, int64_t sA, int64_t sB, int64_t sC, uint32_t a_bytes, uint32_t b_bytes) {
  constexpr int kRows = 32 * (TM + TN);
  constexpr int kRing = ring_depth<TM, TN>();
  __shared__ __attribute__((aligned(1024))) u32x4 ring[kRing][kRows];
  const int lane = threadIdx.x;
  const int r32 = lane & 31, g = lane >> 5;
  const int64_t bz = blockIdx.z;
  const int64_t m_base = static_cast<int64_t>(blockIdx.y) * (32 * TM);
  const int64_t n_base = static_cast<int64_t>(blockIdx.x) * (32 * TN);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(A + bz * sA), 0, a_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(B + bz * sB), 0, b_bytes, kRsrcWord3);

  constexpr int kGroups = kRows / 64;
  uint32_t row_off[kGroups];
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    const int r = 64 * q + lane;
    if (r < 32 * TM) {
      const int64_t m = m_base + r;
      row_off[q] = m < M ? static_cast<uint32_t>(m * lda * 4) : kOOB;
    } else {
      const int64_t n = n_base + (r - 32 * TM);
      row_off[q] = n < N ? static_cast<uint32_t>(n * ldb * 4) : kOOB;
    }
  }
  const int64_t n_stages = (KW + kStageW - 1) / kStageW;
  auto issue = [&](int64_t st, int buf) {
    const bool live = st < n_stages;
    const uint32_t d = static_cast<uint32_t>(st * kStageW * 4);
#pragma unroll
    for (int q = 0; q < kGroups; ++q) {
      const bool is_a = 64 * q < 32 * TM;
      const uint32_t off = (live && row_off[q] != kOOB) ? row_off[q] + d : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? ra : rb, (lds_ptr_t)&ring[buf][64 * q], 16,
                                               off, 0, 0, 0);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  int rowpop[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) rowpop[t] = 0;

  // words g and g+2 of each row of stage st; the last stage clears words
  // past KW and masks the bits past K (uniform branch)
  auto read_stage = [&](u32x2 (&a)[TM], u32x2 (&b)[TN], int64_t st, int rb_) {
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const uint32_t* p = reinterpret_cast<const uint32_t*>(&ring[rb_][t * 32 + r32]) + g;
      a[t] = u32x2{p[0], p[2]};
    }
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const uint32_t* p = reinterpret_cast<const uint32_t*>(&ring[rb_][32 * TM + t * 32 + r32]) + g;
      b[t] = u32x2{p[0], p[2]};
    }
    if (st == n_stages - 1) {
      const int64_t w0 = st * kStageW;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t wi = w0 + g + 2 * h;
        const uint32_t keep = wi < KW - 1 ? 0xFFFFFFFFu : (wi == KW - 1 ? last_mask : 0u);
#pragma unroll
        for (int t = 0; t < TM; ++t) a[t][h] &= keep;
#pragma unroll
        for (int t = 0; t < TN; ++t) b[t][h] &= keep;
      }
    }
  };
  auto unpack = [&](i32x8 (&fa)[TM], i32x8 (&fb)[TN], const u32x2 (&a)[TM],
                    const u32x2 (&b)[TN], int h) {
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      fa[t] = expand_f4_a(a[t][h]);
      if constexpr (SIGNED) rowpop[t] += __builtin_popcount(a[t][h]);
    }
#pragma unroll
    for (int t = 0; t < TN; ++t) fb[t] = expand_f4_b(b[t][h]);
  };
  auto mfmas = [&](const i32x8 (&fa)[TM], const i32x8 (&fb)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb[j], acc[i][j], 4, 4,
                                                                     0, 127, 0, 127);
  };

  // Ring protocol: stage s sits in slot s % kRing.  Iteration s reads the
  // words of stage s+1 and refills the slot of stage s-1, whose words were
  // consumed in iteration s-2.
#pragma unroll
  for (int p = 0; p < kRing - 1; ++p) issue(p, p);
  u32x2 wa[TM], wb[TN];
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kGroups * (kRing - 2)) : "memory");
  read_stage(wa, wb, 0, 0);
  i32x8 fa[TM], fb[TN];
  unpack(fa, fb, wa, wb, 0);
  int slot_next = 1 % kRing, slot_fill = kRing - 1;  // slots of stages s+1, s+kRing-1
  for (int64_t s = 0; s < n_stages; ++s) {
    // stage s+1 has landed once at most the kRing-3 stages after it are
    // outstanding (kGroups loads each; stage s+kRing-1 was issued last)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kGroups * (kRing - 3)) : "memory");
    u32x2 na[TM], nb[TN];
    read_stage(na, nb, s + 1, slot_next);  // past the last stage: zero-filled loads, unused
    issue(s + kRing - 1, slot_fill);
    slot_next = slot_next + 1 == kRing ? 0 : slot_next + 1;
    slot_fill = slot_fill + 1 == kRing ? 0 : slot_fill + 1;
    // k-step 0 of stage s, with k-step 1 unpacked beside it
    i32x8 ga[TM], gb[TN];
    unpack(ga, gb, wa, wb, 1);
    mfmas(fa, fb);
    // k-step 1 of stage s, with k-step 0 of stage s+1 unpacked beside it
    unpack(fa, fb, na, nb, 0);
    mfmas(ga, gb);
#pragma unroll
    for (int t = 0; t < TM; ++t) wa[t] = na[t];
#pragma unroll
    for (int t = 0; t < TN; ++t) wb[t] = nb[t];
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (SIGNED) {
    // the last pass unpacked (and counted) k-step 0 of the stage past the end
#pragma unroll
    for (int t = 0; t < TM; ++t) rowpop[t] -= __builtin_popcount(wa[t][0]);
  }

  // a lane counted the words of its half; the row's count is the pair's sum
  if constexpr (SIGNED) {
#pragma unroll
    for (int t = 0; t < TM; ++t) rowpop[t] += __shfl_xor(rowpop[t], 32, 64);
  }
  store_tile<SIGNED, OUT_F32, TM, TN>(acc, rowpop, static_cast<uint32_t*>(Cv) + bz * sC, M, N, ldc,
                                      m_base, n_base, lane);
}

// 64x128 wave tiles, two waves per SIMD: 8192x4096x4096 in 111 us against
// 121 us for one 128x128 wave per SIMD (its int32 stores could not overlap
// MFMA work) and 122 us for 128x64.
template <bool SIGNED, bool OUT_F32, bool F4, int TM = 2, int TN = 4>
int launch_mfma(const uint32_t* A, const uint32_t* B, void* C, int64_t batch, int64_t M,
                int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t sA,
                int64_t sB, int64_t sC, hipStream_t stream) {
  const int64_t KW = (K + 31) / 32;
  const uint32_t last_mask = (K % 32) ? ((1u << (K % 32)) - 1u) : 0xFFFFFFFFu;
  const int64_t gx = (N + 32 * TN - 1) / (32 * TN), gy = (M + 32 * TM - 1) / (32 * TM);
  if (gx > 0x7FFFFFFFll || gy > 65535 || batch > 65535) return SNNK_EUNSUPPORTED;
  // byte offsets within one batch's operand are 32-bit (buffer descriptors)
  const int64_t a_bytes = ((M - 1) * lda + KW) * 4, b_bytes = ((N - 1) * ldb + KW) * 4;
  if (a_bytes + 16 > kOOB || b_bytes + 16 > kOOB) return SNNK_EUNSUPPORTED;
  if (!aligned(A, 4) || !aligned(B, 4)) return SNNK_EALIGN;
  if constexpr (F4)
    hipLaunchKernelGGL((bgemm_f4_kernel<SIGNED, OUT_F32, TM, TN>), dim3(gx, gy, batch), dim3(64),
                       0, stream, A, B, C, M, N, KW, last_mask, lda, ldb, ldc, sA, sB, sC,
                       static_cast<uint32_t>(a_bytes), static_cast<uint32_t>(b_bytes));
  else
    hipLaunchKernelGGL((bgemm_mfma_kernel<SIGNED, OUT_F32, TM, TN>), dim3(gx, gy, batch), dim3(64),
                       0, stream, A, B, C, M, N, KW, last_mask, lda, ldb, ldc, sA, sB, sC,
                       static_cast<uint32_t>(a_bytes), static_cast<uint32_t>(b_bytes));
  return launch_status();
}

}  // namespace
}  // namespace snnk

using namespace snnk;

extern "C" int snnk_binary_gemm(const uint32_t* A, const uint32_t* B, void* C, int32_t c_dtype,
                                int64_t batch, int64_t M, int64_t N, int64_t K,
                                int64_t lda, int64_t ldb, int64_t ldc,
                                int64_t stride_a, int64_t stride_b, int64_t stride_c,
                                int32_t signed_w, int32_t algo, void* stream) {
  if (batch < 0 || M < 0 || N < 0 || K < 0) return SNNK_EINVAL;
  if (batch == 0 || M == 0 || N == 0) return SNNK_OK;
  if (A == nullptr || B == nullptr || C == nullptr) return SNNK_EINVAL;
  if (c_dtype != SNNK_I32 && c_dtype != SNNK_F32) return SNNK_EINVAL;
  const int64_t KW = (K + 31) / 32;
  if (lda < KW || ldb < KW || ldc < N) return SNNK_EINVAL;
  if (batch > 1 && (stride_a < M * lda || stride_b < N * ldb || stride_c < M * ldc))
    return SNNK_EINVAL;
  if (K > (1ll << 30)) return SNNK_EUNSUPPORTED;  // int32 counts
  hipStream_t s = static_cast<hipStream_t>(stream);
  // fp4 MFMA for GEMM-sized problems (fp32 counts are exact below 2^24)
  if (algo == SNNK_BGEMM_AUTO)
    algo = (M >= 128 && N >= 128 && K >= 128) ? (K < (1ll << 24) ? SNNK_BGEMM_MFMA_F4 : SNNK_BGEMM_MFMA_I8)
                                             : SNNK_BGEMM_POPC;
  if (algo == SNNK_BGEMM_POPC)
    return popcount_gemm(A, B, C, c_dtype, batch, M, N, K, lda, ldb, ldc, stride_a, stride_b,
                         stride_c, signed_w ? 1 : 0, s);
  if (algo != SNNK_BGEMM_MFMA_I8 && algo != SNNK_BGEMM_MFMA_F4) return SNNK_EINVAL;
  if (K == 0) {  // no products: fall through the popcount kernel which writes zeros
    return popcount_gemm(A, B, C, c_dtype, batch, M, N, K, lda, ldb, ldc, stride_a, stride_b,
                         stride_c, signed_w ? 1 : 0, s);
  }
  if (algo == SNNK_BGEMM_MFMA_F4 && K >= (1ll << 24)) return SNNK_EUNSUPPORTED;  // fp32 counts
  const int sel = (signed_w ? 4 : 0) | (c_dtype == SNNK_F32 ? 2 : 0) | (algo == SNNK_BGEMM_MFMA_F4 ? 1 : 0);
  // fp4: 128x128 wave tiles (one wave per SIMD, 256 accumulator registers,
  // fewer unpacking ops per MFMA) once they still give every SIMD a wave
  const bool big = batch * ((M + 127) / 128) * ((N + 127) / 128) >= 1024;
#define SNNK_BGEMM_LAUNCH(S, F, X)                                                               \
  ((X && big) ? launch_mfma<S, F, X, 4, 4>(A, B, C, batch, M, N, K, lda, ldb, ldc, stride_a,     \
                                           stride_b, stride_c, s)                                \
              : launch_mfma<S, F, X>(A, B, C, batch, M, N, K, lda, ldb, ldc, stride_a, stride_b, \
                                     stride_c, s))
  switch (sel) {
    case 0: return SNNK_BGEMM_LAUNCH(false, false, false);
    case 1: return SNNK_BGEMM_LAUNCH(false, false, true);
    case 2: return SNNK_BGEMM_LAUNCH(false, true, false);
    case 3: return SNNK_BGEMM_LAUNCH(false, true, true);
    case 4: return SNNK_BGEMM_LAUNCH(true, false, false);
    case 5: return SNNK_BGEMM_LAUNCH(true, false, true);
    case 6: return SNNK_BGEMM_LAUNCH(true, true, false);
    default: return SNNK_BGEMM_LAUNCH(true, true, true);
  }
#undef SNNK_BGEMM_LAUNCH
}
