// Bit packing of {0,1} spikes and the VALU popcount binary GEMM (gfx950).
//
// Packing convention (snn_compiler/kernels/attention.py:195-214 and
// snn_compiler/explore/attention/phase6b_bitpack.py:35-46): element k of a
// packed row is bit k%32 of word k/32, least-significant bit first; bits past
// K in the last word are zero.
//
// Popcount GEMM (snn_compiler/kernels/attention.py:217-233 generalised):
//   C[b][m][n] = sum_w popc(A[b][m][w] & B[b][n][w])            (unsigned)
//   C[b][m][n] = 2*sum_w popc(A & B) - sum_w popc(A[b][m][w])    (signed)
// One v_bcnt_u32_b32 (popcount with accumulate) and one v_and_b32 per 32
// binary multiply-accumulates.
#include "snnk_common.h"

namespace snnk {
namespace {

// ---------------------------------------------------------------------------
// pack: K contiguous (stride_k == 1) with rows that are not 16-byte aligned.
// One wave packs 64 consecutive elements of one row per ballot; a wave walks
// 8 such chunks (512 elements).
// ---------------------------------------------------------------------------
template <typename Raw>
__device__ __forceinline__ bool nz(Raw v);
template <> __device__ __forceinline__ bool nz<float>(float v) { return v != 0.0f; }
template <> __device__ __forceinline__ bool nz<uint16_t>(uint16_t v) { return (v & 0x7FFFu) != 0; }
template <> __device__ __forceinline__ bool nz<uint8_t>(uint8_t v) { return v != 0; }

constexpr int kPackChunks = 8;  // 64-element chunks per wave

template <typename Raw>
__global__ __launch_bounds__(256) void pack_contig_kernel(
    const Raw* __restrict__ src, uint32_t* __restrict__ dst, int64_t batch, int64_t rows,
    int64_t K, int64_t stride_b, int64_t stride_r, int64_t KW) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int64_t chunks_per_row = (K + 64 * kPackChunks - 1) / (64 * kPackChunks);
  const int64_t row = wave / chunks_per_row;  // flattened (b, r)
  if (row >= batch * rows) return;
  const int64_t cr = wave - row * chunks_per_row;
  const int64_t b = row / rows, r = row - b * rows;
  const Raw* s = src + b * stride_b + r * stride_r;
  uint32_t* d = dst + row * KW;
  const int64_t k_base = cr * 64 * kPackChunks;
  bool bitv[kPackChunks];
#pragma unroll
  for (int c = 0; c < kPackChunks; ++c) {
    const int64_t k = k_base + c * 64 + lane;
    bitv[c] = (k < K) ? nz<Raw>(s[k]) : false;
  }
#pragma unroll
  for (int c = 0; c < kPackChunks; ++c) {
    const uint64_t m = __ballot(bitv[c]);
    const int64_t w0 = (k_base + c * 64) >> 5;
    if (lane < 2 && w0 + lane < KW)
      d[w0 + lane] = static_cast<uint32_t>(m >> (32 * lane));
  }
}

// ---------------------------------------------------------------------------
// pack: K contiguous, rows 16-byte aligned.  One thread builds one word from
// its 32 elements with 16-byte loads (2, 4 or 8 of them for 1-, 2- and
// 4-byte elements); neighbouring threads take neighbouring words, so a
// wave's loads cover one contiguous span and its word stores 256 contiguous
// bytes.  The last word of a row with K % 32 != 0 reads element by element.
// ---------------------------------------------------------------------------
// Bit i of the result: element i of the 16 bytes in v is nonzero (the
// element order of nz).
template <typename Raw>
__device__ __forceinline__ uint32_t nz_bits(u32x4 v);
template <> __device__ __forceinline__ uint32_t nz_bits<uint8_t>(u32x4 v) {
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = v[i];
    // bit 7 of each byte: the byte is nonzero ((b & 0x7F) + 0x7F carries
    // into bit 7 unless the low seven bits are zero; the OR adds bit 7)
    const uint32_t m = (((d & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | d) & 0x80808080u;
    // bits 0, 8, 16, 24 -> bits 28..31 in byte order
    bits |= (((m >> 7) * 0x10204080u) >> 28) << (4 * i);
  }
  return bits;
}
template <> __device__ __forceinline__ uint32_t nz_bits<uint16_t>(u32x4 v) {
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bits |= ((v[i] & 0x00007FFFu) != 0 ? 1u : 0u) << (2 * i);
    bits |= ((v[i] & 0x7FFF0000u) != 0 ? 1u : 0u) << (2 * i + 1);
  }
  return bits;
}
template <> __device__ __forceinline__ uint32_t nz_bits<float>(u32x4 v) {
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) bits |= ((v[i] & 0x7FFFFFFFu) != 0 ? 1u : 0u) << i;  // -0 is zero
  return bits;
}

template <typename Raw>
__global__ __launch_bounds__(256) void pack_word_kernel(
    const Raw* __restrict__ src, uint32_t* __restrict__ dst, int64_t n_words, int64_t rows,
    int64_t K, int64_t stride_b, int64_t stride_r, int64_t KW) {
  constexpr int V = 16 / sizeof(Raw);  // elements per 16-byte load
  constexpr int L = 32 / V;            // loads per word
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= n_words) return;
  const int64_t row = gid / KW, w = gid - row * KW;  // flattened (b, r), word
  const int64_t b = row / rows, r = row - b * rows;
  const Raw* s = src + b * stride_b + r * stride_r;
  const int64_t k0 = w * 32;
  uint32_t word = 0;
  if (k0 + 32 <= K) {
    const u32x4* p = reinterpret_cast<const u32x4*>(s + k0);
    u32x4 v[L];
#pragma unroll
    for (int i = 0; i < L; ++i) v[i] = __builtin_nontemporal_load(p + i);
#pragma unroll
    for (int i = 0; i < L; ++i) word |= nz_bits<Raw>(v[i]) << (i * V);
  } else {
    const int n = static_cast<int>(K - k0);
    for (int j = 0; j < n; ++j) word |= (nz<Raw>(s[k0 + j]) ? 1u : 0u) << j;
  }
  dst[gid] = word;
}

// ---------------------------------------------------------------------------
// pack: K strided.  One thread builds one word from 32 strided elements;
// neighbouring threads take neighbouring rows so every read is coalesced
// when stride_r == 1 (the reference's [TBH, N, D] -> [TBH, D, W] case).
// ---------------------------------------------------------------------------
template <typename Raw>
__global__ __launch_bounds__(256) void pack_strided_kernel(
    const Raw* __restrict__ src, uint32_t* __restrict__ dst, int64_t batch, int64_t rows,
    int64_t K, int64_t stride_b, int64_t stride_r, int64_t stride_k, int64_t KW) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  // thread order: (b, w, r) with r fastest
  const int64_t per_b = KW * rows;
  if (tid >= batch * per_b) return;
  const int64_t b = tid / per_b;
  const int64_t rem = tid - b * per_b;
  const int64_t w = rem / rows, r = rem - w * rows;
  const Raw* s = src + b * stride_b + r * stride_r;
  uint32_t word = 0;
  const int64_t k0 = w * 32;
  const int n = static_cast<int>((K - k0) < 32 ? (K - k0) : 32);
  for (int j = 0; j < n; ++j) word |= (nz<Raw>(s[(k0 + j) * stride_k]) ? 1u : 0u) << j;
  dst[(b * rows + r) * KW + w] = word;
}

// ---------------------------------------------------------------------------
// pack: K strided over contiguous rows (stride_r == 1, rows % 4 == 0, every
// 4-row group aligned).  A thread builds the words of 4 adjacent rows with
// one 4-element load per k (4, 8 or 16 bytes), neighbouring threads on
// neighbouring row groups, so a wave's load covers one contiguous span.
// ---------------------------------------------------------------------------
template <typename Raw> struct Quad;
template <> struct Quad<uint8_t> { typedef uint32_t type; };
template <> struct Quad<uint16_t> { typedef u32x2 type; };
template <> struct Quad<float> { typedef u32x4 type; };

// bit i (i < 4): element i of the 4 loaded is nonzero
__device__ __forceinline__ uint32_t nz4(uint32_t v) {  // 4 bytes
  const uint32_t m = (((v & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | v) & 0x80808080u;
  return ((m >> 7) * 0x10204080u) >> 28;
}
__device__ __forceinline__ uint32_t nz4(u32x2 v) {  // 4 x 16-bit
  return ((v[0] & 0x7FFFu) != 0 ? 1u : 0u) | ((v[0] & 0x7FFF0000u) != 0 ? 2u : 0u) |
         ((v[1] & 0x7FFFu) != 0 ? 4u : 0u) | ((v[1] & 0x7FFF0000u) != 0 ? 8u : 0u);
}
__device__ __forceinline__ uint32_t nz4(u32x4 v) {  // 4 x fp32
  return ((v[0] & 0x7FFFFFFFu) != 0 ? 1u : 0u) | ((v[1] & 0x7FFFFFFFu) != 0 ? 2u : 0u) |
         ((v[2] & 0x7FFFFFFFu) != 0 ? 4u : 0u) | ((v[3] & 0x7FFFFFFFu) != 0 ? 8u : 0u);
}

template <typename Raw>
__global__ __launch_bounds__(256) void pack_strided4_kernel(
    const Raw* __restrict__ src, uint32_t* __restrict__ dst, int64_t batch, int64_t rows,
    int64_t K, int64_t stride_b, int64_t stride_k, int64_t KW) {
  typedef typename Quad<Raw>::type Q;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t rq = rows / 4;
  const int64_t per_b = KW * rq;  // thread order: (b, w, row group) with the group fastest
  if (tid >= batch * per_b) return;
  const int64_t b = tid / per_b;
  const int64_t rem = tid - b * per_b;
  const int64_t w = rem / rq, r0 = (rem - w * rq) * 4;
  const Raw* s = src + b * stride_b + r0;
  const int64_t k0 = w * 32;
  const int n = static_cast<int>((K - k0) < 32 ? (K - k0) : 32);
  uint32_t word[4] = {0u, 0u, 0u, 0u};
#pragma unroll 8
  for (int j = 0; j < n; ++j) {
    const uint32_t q = nz4(__builtin_nontemporal_load(reinterpret_cast<const Q*>(s + (k0 + j) * stride_k)));
#pragma unroll
    for (int i = 0; i < 4; ++i) word[i] |= ((q >> i) & 1u) << j;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[(b * rows + r0 + i) * KW + w] = word[i];
}

template <typename Raw>
int launch_pack(const void* src, uint32_t* dst, int64_t batch, int64_t rows, int64_t K,
                int64_t sb, int64_t sr, int64_t sk, hipStream_t stream) {
  const int64_t KW = (K + 31) / 32;
  const Raw* s = static_cast<const Raw*>(src);
  const int64_t eb = static_cast<int64_t>(sizeof(Raw));
  // every row starts on a 16-byte boundary (a stride of a dimension of
  // extent 1 is never applied)
  const bool rows_aligned = aligned(s, 16) && (rows == 1 || ((sr * eb) & 15) == 0) &&
                            (batch == 1 || ((sb * eb) & 15) == 0);
  if (sk == 1 && rows_aligned) {
    const int64_t n_words = batch * rows * KW;
    const int64_t blocks = (n_words + 255) / 256;
    if (blocks > 0x7FFFFFFFll) return SNNK_EUNSUPPORTED;
    hipLaunchKernelGGL(pack_word_kernel<Raw>, dim3(blocks), dim3(256), 0, stream,
                       s, dst, n_words, rows, K, sb, sr, KW);
  } else if (sk == 1) {
    const int64_t cpr = (K + 64 * kPackChunks - 1) / (64 * kPackChunks);
    const int64_t waves = batch * rows * cpr;
    const int64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7FFFFFFFll) return SNNK_EUNSUPPORTED;
    hipLaunchKernelGGL(pack_contig_kernel<Raw>, dim3(blocks), dim3(256), 0, stream,
                       s, dst, batch, rows, K, sb, sr, KW);
  } else if (sr == 1 && rows % 4 == 0 && aligned(s, 4 * eb) && ((sk * eb) % (4 * eb)) == 0 &&
             (batch == 1 || ((sb * eb) % (4 * eb)) == 0)) {
    const int64_t threads = batch * (rows / 4) * KW;
    const int64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7FFFFFFFll) return SNNK_EUNSUPPORTED;
    hipLaunchKernelGGL(pack_strided4_kernel<Raw>, dim3(blocks), dim3(256), 0, stream,
                       s, dst, batch, rows, K, sb, sk, KW);
  } else {
    const int64_t threads = batch * rows * KW;
    const int64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7FFFFFFFll) return SNNK_EUNSUPPORTED;
    hipLaunchKernelGGL(pack_strided_kernel<Raw>, dim3(blocks), dim3(256), 0, stream,
                       s, dst, batch, rows, K, sb, sr, sk, KW);
  }
  return launch_status();
}

// ---------------------------------------------------------------------------
// VALU popcount GEMM.  Block = 256 threads as a 16x16 grid; each thread owns
// TM x TN outputs (rows ty + 16*i, cols tx + 16*j, so LDS reads of a row
// group are conflict-free broadcasts).  KWB packed words of A and B are
// staged in LDS per iteration.
// ---------------------------------------------------------------------------
constexpr int kKWB = 8;

template <int TM, int TN, bool OUT_F32>
__global__ __launch_bounds__(256) void popc_gemm_kernel(
    const uint32_t* __restrict__ A, const uint32_t* __restrict__ B, void* __restrict__ Cv,
    int64_t M, int64_t N, int64_t KW, uint32_t last_mask, int64_t lda, int64_t ldb,
    int64_t ldc, int64_t sA, int64_t sB, int64_t sC, int signed_w) {
  constexpr int BM = 16 * TM, BN = 16 * TN;
  __shared__ uint32_t sa[kKWB][BM + 1];
  __shared__ uint32_t sb[kKWB][BN + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t bz = blockIdx.z;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN;
  A += bz * sA;
  B += bz * sB;

  uint32_t acc[TM][TN];
  uint32_t rowpop[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    rowpop[i] = 0;
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = 0;
  }

  for (int64_t w0 = 0; w0 < KW; w0 += kKWB) {
    // stage: thread t loads words for (row, word) pairs, row-major over the tile
    for (int e = threadIdx.x; e < BM * kKWB; e += 256) {
      const int r = e / kKWB, w = e - r * kKWB;
      const int64_t gm = m0 + r, gw = w0 + w;
      uint32_t v = 0;
      if (gm < M && gw < KW) {
        v = A[gm * lda + gw];
        if (gw == KW - 1) v &= last_mask;
      }
      sa[w][r] = v;
    }
    for (int e = threadIdx.x; e < BN * kKWB; e += 256) {
      const int r = e / kKWB, w = e - r * kKWB;
      const int64_t gn = n0 + r, gw = w0 + w;
      uint32_t v = 0;
      if (gn < N && gw < KW) {
        v = B[gn * ldb + gw];
        if (gw == KW - 1) v &= last_mask;
      }
      sb[w][r] = v;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kKWB; ++w) {
      uint32_t a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = sa[w][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = sb[w][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        rowpop[i] += __builtin_popcount(a[i]);
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] += __builtin_popcount(a[i] & b[j]);
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t gm = m0 + ty + 16 * i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t gn = n0 + tx + 16 * j;
      if (gn >= N) continue;
      int32_t c = static_cast<int32_t>(acc[i][j]);
      if (signed_w) c = 2 * c - static_cast<int32_t>(rowpop[i]);
      if constexpr (OUT_F32)
        static_cast<float*>(Cv)[bz * sC + gm * ldc + gn] = static_cast<float>(c);
      else
        static_cast<int32_t*>(Cv)[bz * sC + gm * ldc + gn] = c;
    }
  }
}

template <int TM, int TN, bool OUT_F32>
int launch_popc(const uint32_t* A, const uint32_t* B, void* C, int64_t batch, int64_t M,
                int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t sA,
                int64_t sB, int64_t sC, int signed_w, hipStream_t stream) {
  constexpr int BM = 16 * TM, BN = 16 * TN;
  const int64_t KW = (K + 31) / 32;
  const uint32_t last_mask = (K % 32) ? ((1u << (K % 32)) - 1u) : 0xFFFFFFFFu;
  const int64_t gx = (N + BN - 1) / BN, gy = (M + BM - 1) / BM;
  if (gx > 0x7FFFFFFFll || gy > 65535 || batch > 65535) return SNNK_EUNSUPPORTED;
  hipLaunchKernelGGL((popc_gemm_kernel<TM, TN, OUT_F32>), dim3(gx, gy, batch), dim3(256), 0,
                     stream, A, B, C, M, N, KW, last_mask, lda, ldb, ldc, sA, sB, sC, signed_w);
  return launch_status();
}

template <bool OUT_F32>
int popc_dispatch(const uint32_t* A, const uint32_t* B, void* C, int64_t batch, int64_t M,
                  int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t sA,
                  int64_t sB, int64_t sC, int signed_w, hipStream_t s) {
  if (M <= 64 && N <= 64)
    return launch_popc<4, 4, OUT_F32>(A, B, C, batch, M, N, K, lda, ldb, ldc, sA, sB, sC, signed_w, s);
  return launch_popc<8, 8, OUT_F32>(A, B, C, batch, M, N, K, lda, ldb, ldc, sA, sB, sC, signed_w, s);
}

}  // namespace

// Shared with the MFMA binary GEMM (bgemm.hip).
int popcount_gemm(const uint32_t* A, const uint32_t* B, void* C, int32_t c_dtype,
                  int64_t batch, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                  int64_t ldc, int64_t sA, int64_t sB, int64_t sC, int signed_w,
                  hipStream_t s) {
  if (c_dtype == SNNK_F32)
    return popc_dispatch<true>(A, B, C, batch, M, N, K, lda, ldb, ldc, sA, sB, sC, signed_w, s);
  return popc_dispatch<false>(A, B, C, batch, M, N, K, lda, ldb, ldc, sA, sB, sC, signed_w, s);
}

}  // namespace snnk

using namespace snnk;

extern "C" int snnk_pack_bits(const void* src, int32_t src_dtype, uint32_t* dst,
                              int64_t batch, int64_t rows, int64_t K, int64_t stride_b,
                              int64_t stride_r, int64_t stride_k, void* stream) {
  if (batch < 0 || rows < 0 || K < 0) return SNNK_EINVAL;
  if (batch == 0 || rows == 0 || K == 0) return SNNK_OK;
  if (src == nullptr || dst == nullptr || stride_k <= 0) return SNNK_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (src_dtype) {
    case SNNK_F32: return launch_pack<float>(src, dst, batch, rows, K, stride_b, stride_r, stride_k, s);
    case SNNK_BF16:
    case SNNK_F16: return launch_pack<uint16_t>(src, dst, batch, rows, K, stride_b, stride_r, stride_k, s);
    case SNNK_U8: return launch_pack<uint8_t>(src, dst, batch, rows, K, stride_b, stride_r, stride_k, s);
    default: return SNNK_EINVAL;
  }
}
