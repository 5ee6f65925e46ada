// Bit-packed binary GEMM on int8 MFMA (gfx950 v_mfma_i32_32x32x32_i8).
//
//   C[b][m][n] = sum_k A01[m][k] * B01[n][k]                (unsigned)
//   C[b][m][n] = 2 * sum_k A01*B01 - sum_k A01[m][k]         (signed weights)
// with A, B packed along k as uint32 words (bit k%32 of word k/32).
//
// Each wave owns a 128x128 tile of C as 4x4 MFMA 32x32 accumulators and walks
// K in stages of 4 words (128 bits).  Packed words are loaded straight into
// registers one stage ahead; no LDS.  A packed 32-bit word feeds one MFMA
// k-step (32 int8 k values): the lane half g (lane/32) builds its 16 operand
// bytes as the 4 dwords (w >> (4g+s)) & 0x01010101, s = 0..3, i.e. byte b of
// dword s holds bit 4g+s+8b.  A and B operands use this same bit->k
// assignment, so every bit of A meets the matching bit of B in the
// contraction whatever the instruction's internal k order is.
#include "snnk_common.h"

namespace snnk {

int popcount_gemm(const uint32_t* A, const uint32_t* B, void* C, int32_t c_dtype,
                  int64_t batch, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                  int64_t ldc, int64_t sA, int64_t sB, int64_t sC, int signed_w,
                  hipStream_t s);

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kTile = 128;     // per wave, square
constexpr int kStageW = 4;     // packed words per stage

// Four packed words of a row starting at word w0, all inside the row.
template <bool VEC>
__device__ __forceinline__ u32x4 load_full(const uint32_t* row, int64_t w0) {
  if constexpr (VEC) {
    return *reinterpret_cast<const u32x4*>(row + w0);
  } else {
    u32x4 v;
    v[0] = row[w0]; v[1] = row[w0 + 1]; v[2] = row[w0 + 2]; v[3] = row[w0 + 3];
    return v;
  }
}

// The last (partial) stage: words past KW read as 0, the last word masked.
__device__ __forceinline__ u32x4 load_tail(const uint32_t* row, int64_t w0, int64_t KW,
                                           uint32_t last_mask) {
  u32x4 v = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < kStageW; ++j) {
    if (w0 + j < KW) {
      uint32_t x = row[w0 + j];
      v[j] = (w0 + j == KW - 1) ? (x & last_mask) : x;
    }
  }
  return v;
}

__device__ __forceinline__ i32x4 expand(uint32_t w, int g) {
  const uint32_t x = w >> (4 * g);
  i32x4 r;
  r[0] = static_cast<int>(x & 0x01010101u);
  r[1] = static_cast<int>((x >> 1) & 0x01010101u);
  r[2] = static_cast<int>((x >> 2) & 0x01010101u);
  r[3] = static_cast<int>((x >> 3) & 0x01010101u);
  return r;
}

// 4 MFMA k-steps of one stage for the wave's 4x4 accumulator tiles.
template <bool SIGNED>
__device__ __forceinline__ void mfma_stage(i32x16 (&acc)[4][4], const u32x4 (&a)[4],
                                           const u32x4 (&b)[4], int g, int (&rowpop)[4]) {
#pragma unroll
  for (int kk = 0; kk < kStageW; ++kk) {
    i32x4 fa[4], fb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      fa[t] = expand(a[t][kk], g);
      fb[t] = expand(b[t][kk], g);
      if constexpr (SIGNED) rowpop[t] += __builtin_popcount(a[t][kk]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
  }
}

// n_main stages of 4 full words run without guards; a final partial stage
// (KW % 4 != 0, or a masked last word) runs once with guards.
template <bool SIGNED, bool OUT_F32, bool VEC>
__global__ __launch_bounds__(64) void bgemm_mfma_kernel(
    const uint32_t* __restrict__ A, const uint32_t* __restrict__ B, void* __restrict__ Cv,
    int64_t M, int64_t N, int64_t KW, int64_t n_main, int has_tail, uint32_t last_mask,
    int64_t lda, int64_t ldb, int64_t ldc, int64_t sA, int64_t sB, int64_t sC) {
  const int lane = threadIdx.x;
  const int r32 = lane & 31, g = lane >> 5;
  const int64_t bz = blockIdx.z;
  const int64_t m_base = static_cast<int64_t>(blockIdx.y) * kTile;
  const int64_t n_base = static_cast<int64_t>(blockIdx.x) * kTile;
  A += bz * sA;
  B += bz * sB;

  // Rows past M / N read row 0: they only feed outputs that are never stored.
  const uint32_t* arow[4];
  const uint32_t* brow[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t m = m_base + t * 32 + r32, n = n_base + t * 32 + r32;
    arow[t] = A + (m < M ? m : 0) * lda;
    brow[t] = B + (n < N ? n : 0) * ldb;
  }

  i32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;
  int rowpop[4] = {0, 0, 0, 0};

  // Stage s < n_main holds 4 full words; stage n_main (if has_tail) is the
  // guarded partial stage.  The loads of stage s+1 are issued before stage s
  // runs on the MFMA pipe; one MFMA block serves every stage.
  const int64_t n_stages = n_main + has_tail;
  u32x4 a_cur[4], b_cur[4];
  auto load_stage = [&](u32x4 (&a)[4], u32x4 (&b)[4], int64_t st) {
    const int64_t w0 = st * kStageW;
    if (st < n_main) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        a[t] = load_full<VEC>(arow[t], w0);
        b[t] = load_full<VEC>(brow[t], w0);
      }
    } else if (st < n_stages) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        a[t] = load_tail(arow[t], w0, KW, last_mask);
        b[t] = load_tail(brow[t], w0, KW, last_mask);
      }
    }
  };
  load_stage(a_cur, b_cur, 0);
  for (int64_t s = 0; s < n_stages; ++s) {
    u32x4 a_nxt[4], b_nxt[4];
    load_stage(a_nxt, b_nxt, s + 1);
    mfma_stage<SIGNED>(acc, a_cur, b_cur, g, rowpop);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      a_cur[t] = a_nxt[t];
      b_cur[t] = b_nxt[t];
    }
  }

  // Epilogue.  Accumulator register e of lane l holds row 8*(e/4) + 4*g + e%4,
  // column l%32 of its 32x32 tile.
  void* Cb = OUT_F32 ? static_cast<void*>(static_cast<float*>(Cv) + bz * sC)
                     : static_cast<void*>(static_cast<int32_t*>(Cv) + bz * sC);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int rr = 8 * (e >> 2) + 4 * g + (e & 3);
      int rp = 0;
      if constexpr (SIGNED) rp = __shfl(rowpop[i], rr, 64);
      const int64_t m = m_base + i * 32 + rr;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = n_base + j * 32 + r32;
        if (m < M && n < N) {
          int32_t c = acc[i][j][e];
          if constexpr (SIGNED) c = 2 * c - rp;
          if constexpr (OUT_F32)
            __builtin_nontemporal_store(static_cast<float>(c), static_cast<float*>(Cb) + m * ldc + n);
          else
            __builtin_nontemporal_store(c, static_cast<int32_t*>(Cb) + m * ldc + n);
        }
      }
    }
  }
}

template <bool SIGNED, bool OUT_F32>
int launch_mfma(const uint32_t* A, const uint32_t* B, void* C, int64_t batch, int64_t M,
                int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t sA,
                int64_t sB, int64_t sC, hipStream_t stream) {
  const int64_t KW = (K + 31) / 32;
  const uint32_t last_mask = (K % 32) ? ((1u << (K % 32)) - 1u) : 0xFFFFFFFFu;
  const bool has_tail = (KW % kStageW != 0) || (last_mask != 0xFFFFFFFFu);
  const int64_t n_main = has_tail ? KW / kStageW - ((KW % kStageW == 0) ? 1 : 0) : KW / kStageW;
  const int64_t gx = (N + kTile - 1) / kTile, gy = (M + kTile - 1) / kTile;
  if (gx > 0x7FFFFFFFll || gy > 65535 || batch > 65535) return SNNK_EUNSUPPORTED;
  // 16-byte row loads need 16-byte aligned rows
  const bool vec = aligned(A, 16) && aligned(B, 16) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                   (batch == 1 || ((sA % 4 == 0) && (sB % 4 == 0)));
  if (vec)
    hipLaunchKernelGGL((bgemm_mfma_kernel<SIGNED, OUT_F32, true>), dim3(gx, gy, batch), dim3(64),
                       0, stream, A, B, C, M, N, KW, n_main, has_tail ? 1 : 0, last_mask, lda,
                       ldb, ldc, sA, sB, sC);
  else
    hipLaunchKernelGGL((bgemm_mfma_kernel<SIGNED, OUT_F32, false>), dim3(gx, gy, batch), dim3(64),
                       0, stream, A, B, C, M, N, KW, n_main, has_tail ? 1 : 0, last_mask, lda,
                       ldb, ldc, sA, sB, sC);
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
  if (algo == SNNK_BGEMM_AUTO) algo = (M >= 128 && N >= 128 && K >= 128) ? SNNK_BGEMM_MFMA_I8 : SNNK_BGEMM_POPC;
  if (algo == SNNK_BGEMM_POPC)
    return popcount_gemm(A, B, C, c_dtype, batch, M, N, K, lda, ldb, ldc, stride_a, stride_b,
                         stride_c, signed_w ? 1 : 0, s);
  if (algo != SNNK_BGEMM_MFMA_I8) return SNNK_EINVAL;
  const bool f32 = c_dtype == SNNK_F32;
  if (K == 0) {  // no products: fall through the popcount kernel which writes zeros
    return popcount_gemm(A, B, C, c_dtype, batch, M, N, K, lda, ldb, ldc, stride_a, stride_b,
                         stride_c, signed_w ? 1 : 0, s);
  }
  if (signed_w)
    return f32 ? launch_mfma<true, true>(A, B, C, batch, M, N, K, lda, ldb, ldc, stride_a, stride_b, stride_c, s)
               : launch_mfma<true, false>(A, B, C, batch, M, N, K, lda, ldb, ldc, stride_a, stride_b, stride_c, s);
  return f32 ? launch_mfma<false, true>(A, B, C, batch, M, N, K, lda, ldb, ldc, stride_a, stride_b, stride_c, s)
             : launch_mfma<false, false>(A, B, C, batch, M, N, K, lda, ldb, ldc, stride_a, stride_b, stride_c, s);
}
