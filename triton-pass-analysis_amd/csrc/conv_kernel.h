// Kernel template of the fused conv3x3 (stride 1, pad 1) + folded-BN bias + multi-step LIF
// (+ 2x2 max-pool) for gfx950: implicit GEMM on bf16 MFMA
// (v_mfma_f32_32x32x16_bf16) with fp32 accumulation.
//
// Reference path replaced (snn_compiler/nn/modules.py:324-357 ->
// F.conv2d + fused_bias_if_lif at snn_compiler/kernels/fused.py:101-114,
// then a separate nn.MaxPool2d, snn_compiler/zoo/vgg.py:101-105).
//
// Layouts
//   x    [T][B][H][W][Cin]   bf16 (NHWC per step; spikes or real values)
//   w    [Cout][9*Cin]       bf16, k = (kh*3 + kw)*Cin + cin (BN folded)
//   bias [Cout]              fp32 (folded BN shift)
//   out  [T][B][Ho][Wo][Cout] bf16 spikes 0/1   (Ho = H/2 with pooling)
//   pre  [T][B][H][W][Cout]  fp32 conv + bias   (MODE_PREACT, no LIF)
//
// GEMM view: M = T*B*H*W output pixels x steps, N = Cout, K = 9*Cin.
// Row order inside every 32-row MFMA tile is r = 8*q + 4*g + t: two "quads"
// (g = 0, 1) of four pixels (q = 0..3) at four time steps (t = 0..3).  With
// pooling a quad is one 2x2 window (pixel q at dy = q/2, dx = q%2) and maps
// to one pooled pixel; without pooling a quad is four consecutive pixels of
// the flattened (b, y, x) index.  The 32x32 accumulator layout puts rows
// 8*(e/4) + 4*(lane/32) + e%4 in register e of a lane, so each lane holds all
// four time steps of its four pixels for one channel: the LIF recurrence and
// the 2x2 max (an OR of spikes) run in registers and only spikes are stored.
// Longer T runs in chunks of 4 steps with the membrane kept in registers.
//
// A block is WM x WN x KS waves.  Each wave owns TM x TN accumulator tiles;
// the KS wave groups take interleaved 64-wide K stages of the same output
// tile (group g: stages g, g+KS, ...) and are summed through LDS before the
// epilogue (split-K for the small late layers); blocks may also split K
// across the grid (partials in a workspace).  Operand stages stream through
// an NBUF-deep LDS ring filled by direct global->LDS buffer loads; each
// lane's source offsets are rebuilt only when the stage's tap changes.
#pragma once

#include <algorithm>
#include <cstddef>
#include <type_traits>

#include "snnk_common.h"

namespace snnk {


typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kKS = 64;           // K per stage
constexpr int kRow = kKS;         // LDS row pitch in bf16 (128 B, eight 16-byte chunks)
constexpr int kRowBytes = kRow * 2;
constexpr int kDmaRows = 1024 / kRowBytes;  // rows filled by one wave-wide 16-byte load
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format
// buffer-access cache policy sc0 | sc1: system-coherent, through to memory
// past the XCD's L2 (the split-K partial sums of blocks on other XCDs)
constexpr int kSystemCoherent = 17;
// Offset base past every operand: kFar plus any stage delta (< 2^31) stays
// below 2^32 and at or past the end of an operand of at most kFar bytes, so
// such a load reads zeros (padding taps, rows past the end, steps past T,
// columns past Cout, the half of a last stage past K).
constexpr uint32_t kFar = 0x80000000u;

// Wait until at most N of this wave's vector-memory loads are outstanding,
// then meet the other waves of the block.  Written out so that no release
// fence (and its full vmcnt(0) wait) is attached to the barrier.
template <int N>
__device__ __forceinline__ void wait_vmcnt_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// 16-byte chunk c of LDS row r is stored at chunk c ^ key(r).  gfx950 serves
// a ds_read_b128 16 lanes per pass over 64 four-byte banks; the fragment
// reads (16 consecutive rows, one chunk column) then hit 16 distinct 16-byte
// bank groups, and the key is also conflict-free for 8-lane passes.  It
// depends on row bits 0-3 only, so 32-row fragment tiles share it.
__device__ __forceinline__ int swz_key(int r) { return ((r >> 1) ^ (r << 2)) & 7; }
__device__ __forceinline__ int swz(int r, int c) { return c ^ swz_key(r); }

// MODE_MEAN (Linear only): fp32 (x W^T + b) averaged over the T steps,
// out [R][N], for a classifier head whose logits are read as their mean over T.
enum { MODE_LIF = 0, MODE_PREACT = 1, MODE_MEAN = 2 };

struct ConvArgs {
  const uint16_t* x;
  const uint16_t* w;
  const float* bias;
  uint16_t* out;
  float* pre;
  int T, B, H, W, Cin, Cout, Ho, Wo;
  int n_quads;        // quads in one time step
  int n_stages;       // K / 32
  FastDiv div_cin;
  FastDiv div_howo, div_wo, div_hw, div_w;  // row index -> (b, y, x)
  uint32_t x_tstride_b;  // bytes of one input step (B*H*W*Cin*2)
  uint32_t x_bytes;      // bytes of x (T steps), at most kFar
  uint32_t w_bytes;      // bytes of w, at most kFar
  int64_t o_tstride;     // B*Ho*Wo*Cout
  int tiles_m, tiles_n;  // output tiles along rows (quads) and Cout
  FastDiv div_tiles_m, div_tiles_n;
  // cross-block split-K: `splits` blocks share one output tile, each over
  // `stages_per_split` K stages; partial sums go to `partials`, the last
  // block of a tile (ticket in `tickets`) reduces them in split order
  int splits, stages_per_split;
  float* partials;
  unsigned int* tickets;
  float decay, in_scale, vth, v_reset;
  int soft_reset;
  // spikes out as packed words (bit c%32 of word c/32 of a pixel's channels,
  // o_tstride in words) instead of bf16 0/1; MODE_LIF without column pooling
  int bits_out;
  // without split K: deal output tiles to the XCDs Cout-tile major (each XCD
  // streams its own slice of the weights) instead of row-tile major (each
  // XCD streams its own rows of x); set where the weights are the larger operand
  int n_major;
};

static_assert(offsetof(ConvArgs, x) / 64 == 0 && offsetof(ConvArgs, div_cin) / 64 == 1 &&
                  offsetof(ConvArgs, o_tstride) / 64 == 2 && offsetof(ConvArgs, tickets) / 64 == 3 &&
                  sizeof(ConvArgs) <= 256,
              "the kernel touches one field per 64-byte line of ConvArgs");

// LDS of a resident-weight block (NBUF = 0): every K stage of its BN weight
// rows, 128 bytes per row and stage.
constexpr int kResBytes = 160 * 1024;

template <int WM, int WN, int TM, int TN, int KSPLIT, int NBUF, bool PK = false>
struct Cfg {
  static constexpr int kWaves = WM * WN * KSPLIT;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int BM = WM * TM * 32;
  static constexpr int BN = WN * TN * 32;
  static constexpr int kQuads = BM / 16;                    // quads per block
  // NBUF = 0: resident weights.  The block's BN weight rows stay in LDS for
  // all K (loaded once), and each lane loads the packed spike words of its
  // own A rows straight into registers a few stages ahead: the K loop has no
  // barrier and no LDS ring.  Packed A only, one K group, Cin % 64 == 0 and
  // the block's K stages (all of K, or its share under a cross-block split)
  // times BN rows of 128 bytes within kResBytes.
  static constexpr bool kRes = NBUF == 0;
  static_assert(!kRes || (PK && KSPLIT == 1), "resident weights: packed A, one K group");
  // operand stages arrive by direct-to-LDS loads; the WM*WN waves of a K
  // group share them.  B (and bf16 A): 16 bytes per lane, one wave-wide load
  // filling kDmaRows rows (1 KB).  Packed A (PK): the stage's 64 bits of a
  // row are 8 bytes, 4 per lane, one wave-wide load filling 32 rows.
  static constexpr int kARowBytes = PK ? 8 : kRowBytes;
  static constexpr int kARowsPerSeg = PK ? 32 : kDmaRows;
  static constexpr int kSegA = BM / kARowsPerSeg;
  static constexpr int kSegB = BN / kDmaRows;
  static constexpr int kGroupWaves = WM * WN;
  static_assert(kRes || ((PK || kSegA % kGroupWaves == 0) && kSegB % kGroupWaves == 0),
                "segments must split evenly over a group's waves");
  // per wave: A segments first, then B segments.  Packed A segments may not
  // split evenly: the spare waves load a segment again (same bytes to the
  // same place), so that every wave issues the same number of loads.
  // Resident weights: the TM rows of the lane's accumulator tiles.
  static constexpr int kAPer = kRes ? TM : (kSegA + kGroupWaves - 1) / kGroupWaves;
  static constexpr int kBPer = kRes ? 0 : kSegB / kGroupWaves;
  static constexpr int kSegPer = kAPer + kBPer;
  static constexpr int kAStageBytes = KSPLIT * BM * kARowBytes;  // B follows A in a stage
  static constexpr int kStageBytes = kAStageBytes + KSPLIT * BN * kRowBytes;
  static constexpr int kBuf = NBUF;  // ring of operand stages in LDS
  // (resident weights: the most a block may take; the launch sizes it to
  // the block's K stages)
  static constexpr int kLdsBytes = kRes ? kResBytes : kBuf * kStageBytes;
  // K-group sums: a slot per (group, wave, tile) for the tiles another
  // group finishes
  static constexpr int kRedBytes = KSPLIT > 1 ? KSPLIT * WM * WN * TM * TN * 16 * 64 * 4 : 0;
  static constexpr int kSmem = kLdsBytes > kRedBytes ? kLdsBytes : kRedBytes;
  static_assert(kRes || NBUF >= 2, "ring depth");
  // the LDS the block needs fits the CU's 160 KB (some tiles fit only with
  // packed A: launch_cfg refuses their bf16 form)
  static constexpr bool kFits = kSmem <= 160 * 1024;
  // K stages of the resident weights that fit
  static constexpr int kResStages = kResBytes / (BN * kRowBytes);
};

__device__ __forceinline__ uint16_t spike_bf16(bool s) { return s ? 0x3F80u : 0u; }

// 8 spikes (bits 0..7 of b, LSB first) -> 8 bf16 0/1 in four words.  With
// e = b | b << 15, bits 2i and 2i+1 of b sit at bits 2i and 2i + 16 of e;
// masking those two and multiplying by 0x3F80 >> 2i (exact: 0x3F80, bf16
// 1.0, has seven trailing zeros) puts 0x3F80 in the halves they select.
// Two VALU ops per word (the product stays below 2^24: a 24-bit multiply).
__device__ __forceinline__ u32x4 bits_to_bf16x8(uint32_t b) {
  const uint32_t e = b | (b << 15);
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (e & (0x10001u << (2 * i))) * (0x3F80u >> (2 * i));
  return r;
}

// v of the lane CTRL names within each group of 4 lanes (DPP quad_perm)
template <int CTRL>
__device__ __forceinline__ uint32_t quad_dpp(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// TAPS = 9: 3x3 conv, pad 1.  TAPS = 1: 1x1 conv, i.e. a Linear layer over
// the rows of [T][rows][Cin] (H = 1, W = rows).
template <int TAPS>
__device__ __forceinline__ int tap_dy(int tap) { return TAPS == 9 ? tap / 3 - 1 : 0; }
template <int TAPS>
__device__ __forceinline__ int tap_dx(int tap) { return TAPS == 9 ? tap % 3 - 1 : 0; }

// Waves per SIMD a tile's registers must leave room for.  The packed Linear
// 128 x 64 tile serves the short-K projections over many rows (the SSA
// block's QKV: 1152 blocks over 8192 rows, K = 384): unbounded it takes 152
// registers, 3 waves per SIMD, so only 3 of its 4.5 blocks per CU are
// resident at once; bounded to 4 waves it fits 110 registers without spills
// (16.9 us against 18.0).  A bound of 5 waves (96 registers) ran 16.4 us but
// spilled 28 bytes per lane, 7 MB of scratch writes per launch.
template <int WM, int WN, int TM, int TN, int KSPLIT, int NBUF, int TAPS, bool PK>
constexpr int min_waves_per_simd() {
  return WM == 4 && WN == 1 && TM == 1 && TN == 2 && KSPLIT == 1 && NBUF == 3 && TAPS == 1 && PK
             ? 4 : 1;
}

template <int WM, int WN, int TM, int TN, int KSPLIT, int NBUF, bool POOL, int MODE, int TAPS,
          bool PK>
__global__ __launch_bounds__(64 * WM * WN * KSPLIT,
                             (min_waves_per_simd<WM, WN, TM, TN, KSPLIT, NBUF, TAPS, PK>()))
void conv3x3_kernel(ConvArgs a) {
  using C = Cfg<WM, WN, TM, TN, KSPLIT, NBUF, PK>;
  static_assert(C::kFits, "LDS ring must fit 160 KB");
  unsigned char* smem;
  if constexpr (C::kRes) {
    // resident weights: LDS sized at launch to the block's K stages (BN rows
    // of 128 bytes each), so that a short-K layer fits several blocks per CU
    extern __shared__ __attribute__((aligned(1024))) unsigned char smem_res[];
    smem = smem_res;
  } else {
    __shared__ __attribute__((aligned(1024))) unsigned char smem_ring[C::kSmem];
    smem = smem_ring;
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wave / (WM * WN);
  const int wmn = wave - kg * (WM * WN);
  const int wm = wmn / WN, wn = wmn - wm * WN;
  {
    // One field of each 64-byte line of the arguments, loaded together at
    // entry: on first use the scalar loads would go out one line at a time,
    // each a cold miss (0.2 us off the time to the first operand stage).
    const uint32_t l0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(a.x));
    const uint32_t l1 = a.div_cin.m;
    const uint32_t l2 = static_cast<uint32_t>(a.o_tstride);
    const uint32_t l3 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(a.tickets));
    asm volatile("" ::"s"(l0), "s"(l1), "s"(l2), "s"(l3));
  }
  // Workgroups are dealt to the 8 XCDs round-robin by id; id -> tile is
  // remapped so that each XCD runs one contiguous range of tiles.  Without
  // split-K the range is row-tile major (an XCD's L2 holds its rows'
  // activations) or, for weight-heavy layers (n_major), Cout-tile major; with
  // split-K it is (split, Cout tile) major.  Either way the larger operand
  // is streamed from memory about once rather than once per XCD.
  const int n_mn = a.tiles_m * a.tiles_n;
  const int n_tiles = n_mn * a.splits;
  const int per_xcd = (n_tiles + 7) / 8;
  const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (tile >= n_tiles) return;  // whole workgroup: no barrier is left waiting
  int tm, tn, split;
  // (multiply-high dividers: a runtime integer division is ~30 instructions
  // of straight-line code, fetched cold at the start of every launch)
  if (a.splits == 1) {
    if (a.n_major) {
      tn = static_cast<int>(fdiv(static_cast<uint32_t>(tile), a.div_tiles_m));
      tm = tile - tn * a.tiles_m;
    } else {
      tm = static_cast<int>(fdiv(static_cast<uint32_t>(tile), a.div_tiles_n));
      tn = tile - tm * a.tiles_n;
    }
    split = 0;
  } else {
    const int rest = static_cast<int>(fdiv(static_cast<uint32_t>(tile), a.div_tiles_m));
    tm = tile - rest * a.tiles_m;
    split = static_cast<int>(fdiv(static_cast<uint32_t>(rest), a.div_tiles_n));
    tn = rest - split * a.tiles_n;
  }
  const int mn = tm * a.tiles_n + tn;  // output tile id
  const int quad0 = tm * C::kQuads;
  const int n0 = tn * C::BN;
  // this block's K stages [st_begin, st_end)
  const int st_begin = split * a.stages_per_split;
  const int st_end = min(a.n_stages, st_begin + a.stages_per_split);
  const int HW = a.H * a.W;
  constexpr int kPartFloats = TM * TN * 16 * 64;  // a wave's share of an output tile
  const int K = TAPS * a.Cin;

  // Operands are read through range-checked buffer descriptors: an offset
  // at or past the end returns zeros, which is how padding taps, rows past
  // the last pixel, steps past T and columns past Cout are filled.
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.x), 0, a.x_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.w), 0, a.w_bytes, kRsrcWord3);

  // ---- segment geometry (fixed for the whole kernel) ----------------------
  // A segment q of a group's stage is A rows kDmaRows*q.. (1 KB), B segment
  // q is B rows kDmaRows*q..; wave wmn of the group loads A segments
  // wmn + i*kGroupWaves (i < kAPer) and the same B segments (i < kBPer).
  // Lane l writes row kDmaRows*q + l/8, chunk slot l%8, and so reads source
  // chunk c = slot ^ key(row).  Chunks 0-3 hold k0..k0+31 of the stage, chunks
  // 4-7 k0+32..k0+63: the lane's half is h = c/4, and since key(row) has bit
  // 2 = (q ^ row) & 1, h = h0 ^ (q & 1) with h0 = (slot/4) ^ (l/8 & 1).  With
  // Cin % 64 == 32 the two halves of a stage may fall in different taps.
  const int lrow = lane >> 3, slot = lane & 7;
  const uint32_t h0 = static_cast<uint32_t>((slot >> 2) ^ (lrow & 1));
  uint32_t s_base[C::kSegPer];  // A: bytes of (t, b, y, x) + 16*(c%4); B: bytes of (n, c) or kFar
  uint32_t s_ok[C::kAPer];      // A: bit tap set when the row exists and the tap's source
                                // pixel is inside the image
#pragma unroll
  for (int i = 0; i < C::kSegPer; ++i) {
    if (i < C::kAPer) {
      // packed A: lane l takes row 32*q + l/2, half l%2 (its 4 bytes);
      // resident weights: row l%32 of the wave's accumulator tile i
      const int q = PK ? (wmn + i * C::kGroupWaves) % C::kSegA : wmn + i * C::kGroupWaves;
      const int r = C::kRes ? (wm * TM + i) * 32 + (lane & 31)
                            : PK ? 32 * q + (lane >> 1) : kDmaRows * q + lrow;
      const int rr = r & 31;
      const int pq = rr >> 3, gr = (rr >> 2) & 1, t = rr & 3;
      const int quad = quad0 + (r >> 5) * 2 + gr;
      int b = 0, y = 0, xx = 0;
      const bool row_ok = quad < a.n_quads;
      uint32_t ok = 0;
      if (row_ok) {
        if constexpr (POOL && TAPS == 9) {
          b = static_cast<int>(fdiv(static_cast<uint32_t>(quad), a.div_howo));
          const int r2 = quad - b * a.Ho * a.Wo;
          const int py = static_cast<int>(fdiv(static_cast<uint32_t>(r2), a.div_wo));
          const int px = r2 - py * a.Wo;
          y = 2 * py + (pq >> 1);
          xx = 2 * px + (pq & 1);
        } else {
          const int pix = quad * 4 + pq;
          b = static_cast<int>(fdiv(static_cast<uint32_t>(pix), a.div_hw));
          const int r2 = pix - b * HW;
          y = static_cast<int>(fdiv(static_cast<uint32_t>(r2), a.div_w));
          xx = r2 - y * a.W;
        }
        if constexpr (TAPS == 9) {
          // tap kh*3 + kw reads (y + kh - 1, x + kw - 1)
          const uint32_t vx = (xx > 0 ? 1u : 0u) | 2u | (xx + 1 < a.W ? 4u : 0u);
          ok = (y > 0 ? vx : 0u) | (vx << 3) | (y + 1 < a.H ? vx << 6 : 0u);
        } else {
          ok = 1u;
        }
      }
      const int c = swz(r, slot);
      s_base[i] = static_cast<uint32_t>(t) * a.x_tstride_b +
                  static_cast<uint32_t>(((b * a.H + y) * a.W + xx) * a.Cin) * 2u +
                  (PK ? 0u : (c & 3) * 16u);
      s_ok[i] = ok;
    } else {
      const int n = kDmaRows * (wmn + (i - C::kAPer) * C::kGroupWaves) + lrow;
      const int c = swz(n, slot);
      s_base[i] = n0 + n < a.Cout
                      ? static_cast<uint32_t>(n0 + n) * static_cast<uint32_t>(K) * 2u + c * 16u
                      : kFar;
    }
  }

  // every K group runs n_stages_g ring iterations (their barriers are
  // shared); when the block's K stages do not split evenly over the groups,
  // a group's last one lies past the block's range and is loaded as zeros
  const int n_stages_g = (st_end - st_begin + KSPLIT - 1) / KSPLIT;
  const int n_chunks = (a.T + 3) / 4;

  // With K groups, accumulator tile (i, j) of wave wmn is summed and
  // finished (LIF epilogue, or split-K partials) by the wave wmn of group
  // (i*TN + j) % KSPLIT: the epilogue work of a block is spread over its
  // groups instead of falling to group 0 alone.
  auto mine = [&](int i, int j) __attribute__((always_inline)) {
    return KSPLIT == 1 || (i * TN + j) % KSPLIT == kg;
  };
  // membrane state of the tiles this wave finishes: [TM][TN][4 pixels]
  float v[TM][TN][4];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[i][j][q] = 0.0f;

  const int g_lane = lane >> 5, r_lane = lane & 31;
  // epilogue columns and bias, filled after the first operand loads are on
  // their way (the code before them runs once, from a cold instruction cache)
  float bias_n[TN];
  bool col_ok[TN];

  // Packed spikes of tile (i, j): the 32 columns of a tile are one word of
  // channels, so a wave ballot per (step, pixel) gives the words of both
  // quads (low half: lanes 0-31, quad g = 0; high half: g = 1).  Lane L < 32
  // keeps word L -- (step, pixel, g) = (L/8, L/2 % 4, L%2) -- and stores it;
  // pooled tiles have one pixel per quad and 8 words.  Lanes of a quad past
  // the last take no part in the ballots (they skipped the epilogue).
  auto store_words = [&](uint32_t sbits, int i, int j, int tc) __attribute__((always_inline)) {
    constexpr int kWords = POOL ? 4 : 16;
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < kWords; ++b) {
      const uint64_t m = __builtin_amdgcn_ballot_w64(((sbits >> b) & 1u) != 0);
      if ((lane >> 1) == b) word = (lane & 1) ? static_cast<uint32_t>(m >> 32) : static_cast<uint32_t>(m);
    }
    if (lane < 2 * kWords) {
      const int t = POOL ? lane >> 1 : lane >> 3;
      const int q = POOL ? 0 : (lane >> 1) & 3;
      const int quad = quad0 + (wm * TM + i) * 2 + (lane & 1);
      if (tc * 4 + t < a.T && quad < a.n_quads) {
        const int64_t pix = POOL ? static_cast<int64_t>(quad) : static_cast<int64_t>(quad) * 4 + q;
        reinterpret_cast<uint32_t*>(a.out)[static_cast<int64_t>(tc * 4 + t) * a.o_tstride +
                                           pix * (a.Cout >> 5) + ((n0 + (wn * TN + j) * 32) >> 5)] = word;
      }
    }
  };

  // bias + LIF over the 4 steps of chunk tc (+ 2x2 OR) on the full K sum;
  // the reset rule is a compile-time branch (kSoft) so that each neuron
  // update is add, mul, mul, add, compare, select (+ sub when soft)
  auto lif_epilogue = [&](const f32x16 (&acc)[TM][TN], int tc, auto soft_tag)
                          __attribute__((always_inline)) {
    constexpr bool kSoft = decltype(soft_tag)::value;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int quad = quad0 + (wm * TM + i) * 2 + g_lane;
      if (quad >= a.n_quads) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if (!col_ok[j] || !mine(i, j)) continue;
        const int n = n0 + (wn * TN + j) * 32 + r_lane;
        // TAPS = 1 with POOL: the output keeps one column of every group of
        // four adjacent columns (their OR), Cout / 4 columns per row
        constexpr bool kColPool = POOL && TAPS == 1;
        const int o_cols = kColPool ? a.Cout / 4 : a.Cout;
        uint16_t* o = a.out + static_cast<int64_t>(tc) * 4 * a.o_tstride +
                      (POOL && !kColPool ? static_cast<int64_t>(quad) * a.Cout + n
                                         : static_cast<int64_t>(quad) * 4 * o_cols +
                                               (kColPool ? n / 4 : n));
        // packed output: bit 4t+q (spike of pixel q at step t), or bit t (the
        // pooled OR at step t)
        uint32_t sbits = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (tc * 4 + t >= a.T) break;
          bool any = false;
          bool sp[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float u = __fadd_rn(acc[i][j][q * 4 + t], bias_n[j]);
            const float h = __fadd_rn(__fmul_rn(a.decay, v[i][j][q]), __fmul_rn(a.in_scale, u));
            const bool s = h >= a.vth;
            if constexpr (kSoft) v[i][j][q] = s ? __fsub_rn(h, a.vth) : h;
            else v[i][j][q] = s ? a.v_reset : h;
            sp[q] = s;
            any = any || s;
          }
          if constexpr (!kColPool) {
            if (a.bits_out) {
              if constexpr (POOL) sbits |= any ? 1u << t : 0u;
              else
#pragma unroll
                for (int q = 0; q < 4; ++q) sbits |= sp[q] ? 1u << (4 * t + q) : 0u;
              continue;
            }
          }
          if constexpr (kColPool) {
            // lanes 4k..4k+3 hold adjacent columns of the same rows: OR the
            // 4 pixels' spikes (bit q) over the quad with two DPP exchanges
            uint32_t m = (sp[0] ? 1u : 0u) | (sp[1] ? 2u : 0u) | (sp[2] ? 4u : 0u) | (sp[3] ? 8u : 0u);
            m |= quad_dpp<0xB1>(m);  // lane ^ 1
            m |= quad_dpp<0x4E>(m);  // lane ^ 2
            if ((r_lane & 3) == 0) {
#pragma unroll
              for (int q = 0; q < 4; ++q) o[q * o_cols] = spike_bf16(((m >> q) & 1u) != 0);
            }
          } else if constexpr (POOL) {
            o[0] = spike_bf16(any);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q * a.Cout] = spike_bf16(sp[q]);
          }
          o += a.o_tstride;
        }
        if constexpr (!kColPool) {
          if (a.bits_out) store_words(sbits, i, j, tc);
        }
      }
    }
  };
  // the LIF epilogue, or the fp32 pre-activations, of the tiles this wave finishes
  // (both lambdas are forced inline: a call would move the accumulators to scratch)
  auto epilogue = [&](const f32x16 (&acc)[TM][TN], int tc) __attribute__((always_inline)) {
    if constexpr (MODE == MODE_PREACT) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int quad = quad0 + (wm * TM + i) * 2 + g_lane;
        if (quad >= a.n_quads) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (!col_ok[j] || !mine(i, j)) continue;
          const int n = n0 + (wn * TN + j) * 32 + r_lane;
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int tg = tc * 4 + t;
              if (tg < a.T) {
                const int64_t p = static_cast<int64_t>(quad) * 4 + q;
                a.pre[tg * a.o_tstride + p * a.Cout + n] = __fadd_rn(acc[i][j][q * 4 + t], bias_n[j]);
              }
            }
        }
      }
    } else if constexpr (MODE == MODE_MEAN) {
      // running sum over the steps in v (one chunk of 4 at a time), written
      // as sum / T after the last chunk
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int quad = quad0 + (wm * TM + i) * 2 + g_lane;
        if (quad >= a.n_quads) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (!col_ok[j] || !mine(i, j)) continue;
          const int n = n0 + (wn * TN + j) * 32 + r_lane;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
              if (tc * 4 + t < a.T)
                v[i][j][q] = __fadd_rn(v[i][j][q], __fadd_rn(acc[i][j][q * 4 + t], bias_n[j]));
            if (tc == n_chunks - 1)
              a.pre[(static_cast<int64_t>(quad) * 4 + q) * a.Cout + n] =
                  __fdiv_rn(v[i][j][q], static_cast<float>(a.T));
          }
        }
      }
    } else if (a.soft_reset) {
      lif_epilogue(acc, tc, std::true_type{});
    } else {
      lif_epilogue(acc, tc, std::false_type{});
    }
  };

  // ---- resident weights: one fill, then K loops without barriers ----------
  if constexpr (C::kRes) {
    // fill segment g: weight rows 8*(g % kSegB).. of the block's K stage
    // g / kSegB (global stage st_begin + g / kSegB), one 16-byte chunk per
    // lane, swizzled as in the ring; LDS slot s holds the block's BN rows of
    // its stage s at 128 bytes each
    const int n_seg = (st_end - st_begin) * C::kSegB;
    for (int g = wave; g < n_seg; g += C::kWaves) {
      const int st = g / C::kSegB;
      const int n = 8 * (g - st * C::kSegB) + lrow;
      const uint32_t off = n0 + n < a.Cout
                               ? static_cast<uint32_t>(n0 + n) * static_cast<uint32_t>(K) * 2u +
                                     static_cast<uint32_t>(st_begin + st) * kRowBytes + swz(n, slot) * 16u
                               : kFar;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          wr, (lds_ptr_t)(smem + (st * C::BN + n - lrow) * kRowBytes), 16, off, 0, 0, 0);
    }
  }
  // A rows with resident weights: the 64 spikes of stage s of the lane's row
  // (wm*TM + i)*32 + lane%32 are 8 bytes of packed words, loaded into
  // registers kAhead stages before their MFMAs.  The stage loop is unrolled
  // by kAhead so that each stage has registers of its own (a rotation would
  // wait for every load in flight).
  constexpr int kAhead = 3;
  auto res_k_loop = [&](f32x16 (&acc)[TM][TN], int tc, bool t_ok, uint32_t chunk_off)
                        __attribute__((always_inline)) {
    const int n_st = st_end - st_begin;  // this block's K stages (all of K without a split)
    uint32_t a_off[TM];
    int cur_tap = -1;
    auto load_a = [&](int s, u32x2 (&dst)[TM]) __attribute__((always_inline)) {
      const uint32_t k0 = static_cast<uint32_t>(st_begin + s) * kKS;
      const int tap = static_cast<int>(fdiv(k0, a.div_cin));
      const int cin_lo = static_cast<int>(k0) - tap * a.Cin;
      if (tap != cur_tap) {  // every Cin / 64 stages
        cur_tap = tap;
        const int32_t del = (tap_dy<TAPS>(tap) * a.W + tap_dx<TAPS>(tap)) * a.Cin * 2;
#pragma unroll
        for (int i = 0; i < TM; ++i)
          a_off[i] = t_ok && ((s_ok[i] >> tap) & 1u) ? s_base[i] + static_cast<uint32_t>(del) : kFar;
      }
      const uint32_t da = chunk_off + static_cast<uint32_t>(cin_lo) * 2u;
#pragma unroll
      for (int i = 0; i < TM; ++i)  // packed byte offset: a sixteenth of the bf16 one
        dst[i] = __builtin_amdgcn_raw_buffer_load_b64(xr, static_cast<int>((a_off[i] + da) >> 4), 0, 0);
    };
    auto stage = [&](int s, u32x2 (&pa)[TM]) __attribute__((always_inline)) {
      // expand the four k-slices first; the registers then take stage s + kAhead
      bf16x8 fa[4][TM];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const u32x4 e = bits_to_bf16x8((pa[i][kk >> 1] >> (16 * (kk & 1) + 8 * g_lane)) & 0xFFu);
          __builtin_memcpy(&fa[kk][i], &e, 16);
        }
      if (s + kAhead < n_st) load_a(s + kAhead, pa);
      const uint16_t* sb =
          reinterpret_cast<const uint16_t*>(smem) + (s * C::BN + wn * TN * 32 + r_lane) * kRow;
      bf16x8 fb[2][TN];
      auto read_b = [&](bf16x8 (&dst)[TN], int kk) __attribute__((always_inline)) {
        const int ch = swz(r_lane, kk * 2 + g_lane) * 8;
#pragma unroll
        for (int j = 0; j < TN; ++j) dst[j] = *reinterpret_cast<const bf16x8*>(sb + j * 32 * kRow + ch);
      };
      read_b(fb[0], 0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk + 1 < 4) read_b(fb[(kk + 1) & 1], kk + 1);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk][i], fb[kk & 1][j], acc[i][j], 0, 0, 0);
      }
    };
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    u32x2 ring[kAhead][TM];
#pragma unroll
    for (int d = 0; d < kAhead; ++d)
      if (d < n_st) load_a(d, ring[d]);
    if (tc == 0) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + (wn * TN + j) * 32 + r_lane;
        col_ok[j] = n < a.Cout;
        bias_n[j] = (a.bias && col_ok[j]) ? a.bias[n] : 0.0f;
      }
      wait_vmcnt_barrier<0>();  // the resident weights are in LDS
    }
    for (int s0 = 0; s0 < n_st; s0 += kAhead) {
#pragma unroll
      for (int d = 0; d < kAhead; ++d)
        if (s0 + d < n_st) stage(s0 + d, ring[d]);
    }
  };

  for (int tc = 0; tc < n_chunks; ++tc) {
    // Source offsets of this lane's A segments for the tap pair (tap_lo,
    // tap_hi) of the stage last prepared: kFar where the row, the step or
    // the tap's source pixel does not exist.  A stage then costs one add
    // per segment; the offsets are rebuilt only when the tap pair changes.
    // (the step of this lane's A rows: row & 3, with row 8*q + l/8 -- or
    // 32*q + l/2 for packed A, or lane%32 with resident weights)
    const bool t_ok = tc * 4 + ((C::kRes ? lane : PK ? lane >> 1 : lrow) & 3) < a.T;
    const uint32_t chunk_off = static_cast<uint32_t>(tc) * 4u * a.x_tstride_b;
    f32x16 acc[TM][TN];
    if constexpr (C::kRes) {
      res_k_loop(acc, tc, t_ok, chunk_off);
    } else {
      uint32_t a_off[C::kAPer];
#pragma unroll
      for (int i = 0; i < C::kAPer; ++i) a_off[i] = kFar;
      int cur_lo = -1, cur_hi = -1;

      // wave-uniform addressing of the group's next stage to load.  The
      // group's K stages lie KSPLIT apart, so the next one's tap and first
      // channel follow from the last by an add and a compare (one division
      // at the start of the chunk, none per stage)
      struct StageAddr {
        bool live;        // a stage of the ring loop (later slots are not loaded)
        bool zero_b;      // B reads zeros: a stage past the block's K range
        bool tail;        // the last stage of K % 64 == 32: upper half past K
        uint32_t da, db;  // A: chunk + channel bytes of the lower half; B: bytes of k0
      };
      int nx_sl = 0;                   // group-local index of the next stage
      int nx_sg = st_begin + kg;       // its global K stage
      int nx_tap, nx_cin;              // its tap and first channel: k0 = tap * Cin + cin
      {
        const uint32_t k0 = static_cast<uint32_t>(nx_sg * kKS);
        nx_tap = static_cast<int>(fdiv(k0, a.div_cin));
        nx_cin = static_cast<int>(k0) - nx_tap * a.Cin;
      }
      auto prepare_next = [&]() {
        StageAddr p;
        p.live = nx_sl < n_stages_g;
        p.zero_b = nx_sg >= st_end;
        // (a stage past the K range reads as k0 = 0; its B offsets are kFar)
        const int tap_lo = p.zero_b ? 0 : nx_tap;
        const int cin_lo = p.zero_b ? 0 : nx_cin;
        const uint32_t k0 = p.zero_b ? 0u : static_cast<uint32_t>(nx_sg * kKS);
        const bool wrap = cin_lo + 32 >= a.Cin;  // upper half starts the next tap
        const int tap_hi = tap_lo + (wrap ? 1 : 0);
        p.da = chunk_off + static_cast<uint32_t>(cin_lo) * 2u;
        p.db = k0 * 2u;
        p.tail = static_cast<int>(k0) + 32 >= K;
        if (p.live && p.zero_b) {  // (rare) every A offset past the end as well
          cur_lo = cur_hi = -1;
          p.da = 0;
#pragma unroll
          for (int i = 0; i < C::kAPer; ++i) a_off[i] = kFar;
        } else if (p.live && (tap_lo != cur_lo || tap_hi != cur_hi)) {
          cur_lo = tap_lo;
          cur_hi = tap_hi;
          // byte delta of each half's source pixel, relative to p.da; the upper
          // half sits 32 channels on, or at channel cin_lo + 32 - Cin of the
          // next tap (a tap past the last has no ok bit: zeros)
          const int32_t del_lo = (tap_dy<TAPS>(tap_lo) * a.W + tap_dx<TAPS>(tap_lo)) * a.Cin * 2;
          const int32_t del_hi = (tap_dy<TAPS>(tap_hi) * a.W + tap_dx<TAPS>(tap_hi)) * a.Cin * 2 +
                                 64 - (wrap ? 2 * a.Cin : 0);
#pragma unroll
          for (int i = 0; i < C::kAPer; ++i) {
            const uint32_t h = PK ? static_cast<uint32_t>(lane & 1)
                                  : h0 ^ static_cast<uint32_t>((wmn + i * C::kGroupWaves) & 1);
            const int tap = h ? tap_hi : tap_lo;
            const bool ok = t_ok && ((s_ok[i] >> tap) & 1u);
            a_off[i] = ok ? s_base[i] + static_cast<uint32_t>(h ? del_hi : del_lo) : kFar;
          }
        }
        // step to the group's following stage
        ++nx_sl;
        nx_sg += KSPLIT;
        nx_cin += KSPLIT * kKS;
        while (nx_cin >= a.Cin) {
          nx_cin -= a.Cin;
          ++nx_tap;
        }
        return p;
      };
      // enqueue the direct global->LDS load of segment i of a stage.  A ring
      // slot past the loop is loaded too (never read; its offsets stay inside
      // the operands or read zeros): a branch around each load cost more than
      // the loads, and the waits stay conservative
      auto issue_seg = [&](const StageAddr& p, int i, int buf) {
        unsigned char* stage = smem + buf * C::kStageBytes;
        if (i < C::kAPer) {  // resolved at compile time
          // (the offset goes through a variable: with the sum written in the
          // call, hipcc's host pass drops the kernel's launch stub)
          const uint32_t off = a_off[i] + p.da;
          if constexpr (PK) {
            // packed x: the 32 spikes of this lane's half-row are 4 bytes at a
            // sixteenth of the bf16 offset (past-the-end offsets stay past it)
            const int q = (wmn + i * C::kGroupWaves) % C::kSegA;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (lds_ptr_t)(stage + kg * C::BM * 8 + q * 256), 4, off >> 4, 0, 0, 0);
          } else {
            const int q = wmn + i * C::kGroupWaves;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (lds_ptr_t)(stage + (kg * C::BM + kDmaRows * q) * kRowBytes), 16, off, 0, 0, 0);
          }
        } else {
          const int q = wmn + (i - C::kAPer) * C::kGroupWaves;
          const bool upper = (h0 ^ static_cast<uint32_t>(q & 1)) != 0;
          const uint32_t off = (p.zero_b || (p.tail && upper)) ? kFar : s_base[i] + p.db;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              wr, (lds_ptr_t)(stage + C::kAStageBytes + (kg * C::BN + kDmaRows * q) * kRowBytes),
              16, off, 0, 0, 0);
        }
      };

      // a loop, not unrolled: this code runs once per launch from a cold
      // instruction cache, so one copy of it is fetched instead of NBUF-1
#pragma nounroll
      for (int p = 0; p < C::kBuf - 1; ++p) {
        const StageAddr sp = prepare_next();
#pragma unroll
        for (int i = 0; i < C::kSegPer; ++i) issue_seg(sp, i, p);
      }
      // set-up that no load waits for
      if (tc == 0) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = n0 + (wn * TN + j) * 32 + r_lane;
          col_ok[j] = n < a.Cout;
          bias_n[j] = (a.bias && col_ok[j]) ? a.bias[n] : 0.0f;
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
      constexpr int kSlices = kKS / 16;
      int buf = 0;
      // addressing of the stage the next iteration loads; prepared at the end
      // of the previous iteration, so that after each barrier the fragment
      // reads issue at once instead of behind the scalar stage arithmetic
      StageAddr sp = prepare_next();
      for (int s = 0; s < n_stages_g; ++s) {
        // every ring iteration (and the prologue, per stage) issues kSegPer
        // loads, past the end of K as well, so this wave's loads of stage s
        // are done once at most the kBuf - 2 later stages' loads are
        // outstanding; the barrier publishes every wave's loads and retires
        // the reads of the buffer refilled next
        static_assert(C::kSegPer * (C::kBuf - 2) <= 63, "vmcnt holds 6 bits");
        wait_vmcnt_barrier<C::kSegPer * (C::kBuf - 2)>();
        const int nbuf = buf == 0 ? C::kBuf - 1 : buf - 1;

        const unsigned char* st = smem + buf * C::kStageBytes;
        const uint16_t* sa = reinterpret_cast<const uint16_t*>(st) + (kg * C::BM + wm * TM * 32 + r_lane) * kRow;
        const uint16_t* sb = reinterpret_cast<const uint16_t*>(st + C::kAStageBytes) +
                             (kg * C::BN + wn * TN * 32 + r_lane) * kRow;
        // packed A: the stage's 64 bits of each of this lane's rows; slice kk,
        // half g reads byte 2*kk + g (K values 16*kk + 8*g ..)
        u32x2 pa[TM];
        if constexpr (PK) {
#pragma unroll
          for (int i = 0; i < TM; ++i)
            pa[i] = *reinterpret_cast<const u32x2*>(st + (kg * C::BM + wm * TM * 32 + i * 32 + r_lane) * 8);
        }
        auto read = [&](bf16x8 (&fa)[TM], bf16x8 (&fb)[TN], int kk) {
          // tile rows start at multiples of 32, so the swizzle depends on r_lane only
          const int ch = swz(r_lane, kk * 2 + g_lane) * 8;
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            if constexpr (PK) {
              const u32x4 e = bits_to_bf16x8((pa[i][kk >> 1] >> (16 * (kk & 1) + 8 * g_lane)) & 0xFFu);
              __builtin_memcpy(&fa[i], &e, 16);
            } else {
              fa[i] = *reinterpret_cast<const bf16x8*>(sa + i * 32 * kRow + ch);
            }
          }
#pragma unroll
          for (int j = 0; j < TN; ++j) fb[j] = *reinterpret_cast<const bf16x8*>(sb + j * 32 * kRow + ch);
        };
        // software pipeline over the k-slices: the reads of slice kk+1 and a
        // share of the next stage's loads are in flight while slice kk's MFMAs
        // run (the compiler's own interleaving measured 3-6% faster than
        // scheduling barriers around each MFMA group)
        bf16x8 fa[2][TM], fb[2][TN];
        read(fa[0], fb[0], 0);
#pragma unroll
        for (int kk = 0; kk < kSlices; ++kk) {
          if (kk + 1 < kSlices) read(fa[(kk + 1) & 1], fb[(kk + 1) & 1], kk + 1);
#pragma unroll
          for (int i = 0; i < C::kSegPer; ++i)
            if (i % kSlices == kk) issue_seg(sp, i, nbuf);
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk & 1][i], fb[kk & 1][j], acc[i][j], 0, 0, 0);
        }
        sp = prepare_next();
        buf = buf + 1 == C::kBuf ? 0 : buf + 1;
      }
      // every wave is done reading the ring before LDS is reused
      wait_vmcnt_barrier<0>();
    }

    // ---- split-K reduction through LDS ----------------------------------
    if constexpr (KSPLIT > 1) {
      // Each wave parks the tiles another group finishes in its LDS slots
      // (16-byte pieces, lane-contiguous: conflict-free ds_write_b128 /
      // ds_read_b128), then sums the tiles it finishes in group order,
      // ((g0 + g1) + g2) + ..., each group's four reads issued before its adds
      f32x4* red = reinterpret_cast<f32x4*>(smem);
      auto slot = [&](int g, int i, int j) __attribute__((always_inline)) {
        return red + ((g * WM * WN + wmn) * TM * TN + i * TN + j) * 4 * 64 + lane;
      };
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (mine(i, j)) continue;
          f32x4* dst = slot(kg, i, j);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            dst[q * 64] = f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (!mine(i, j)) continue;
          f32x16 sum;
#pragma unroll
          for (int g = 0; g < KSPLIT; ++g) {
            f32x16 part;
            if (g == kg) {
              part = acc[i][j];
            } else {
              const f32x4* src = slot(g, i, j);
              f32x4 pc[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) pc[q] = src[q * 64];
#pragma unroll
              for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int c = 0; c < 4; ++c) part[4 * q + c] = pc[q][c];
            }
            if (g == 0) {
              sum = part;
            } else {
#pragma unroll
              for (int e = 0; e < 16; ++e) sum[e] += part[e];
            }
          }
          acc[i][j] = sum;
        }
      __syncthreads();
    }

    {
      if (a.splits == 1) {
        epilogue(acc, tc);
      } else {
        // this block's partial sums: 16-byte pieces, system-coherent (written
        // through to memory, past this XCD's L2)
        const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
            a.partials + (static_cast<int64_t>(mn) * a.splits + split) * n_chunks * (C::BM * C::BN),
            0, -1, kRsrcWord3);
        const uint32_t voff = static_cast<uint32_t>(tc * (C::BM * C::BN) + wmn * kPartFloats) * 4u +
                              static_cast<uint32_t>(lane) * 16u;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if (!mine(i, j)) continue;
              const i32x4 v = {__float_as_int(acc[i][j][4 * q]), __float_as_int(acc[i][j][4 * q + 1]),
                               __float_as_int(acc[i][j][4 * q + 2]), __float_as_int(acc[i][j][4 * q + 3])};
              __builtin_amdgcn_raw_buffer_store_b128(v, pr, voff + ((i * TN + j) * 4 + q) * 1024, 0,
                                                     kSystemCoherent);
            }
      }
    }
  }

  // ---- cross-block split-K: the last block of a tile reduces and fires -----
  if (a.splits > 1) {
    // The partials were stored write-through and are read back with
    // system-coherent loads, so no cache-wide fence is needed (an agent-scope
    // fence writes back and invalidates the whole L2 of the XCD): each wave
    // waits for its stores to be acknowledged, then one ticket per block.
    // The operand ring is idle now; its first word carries the ticket result.
    volatile unsigned int* s_last = reinterpret_cast<volatile unsigned int*>(smem);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
      *s_last = __hip_atomic_fetch_add(a.tickets + mn, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) ==
                static_cast<unsigned int>(a.splits - 1);
    __syncthreads();
    if (!*s_last) return;
    {
      // the partial sums of the tiles this wave finishes, read back with
      // system-coherent 16-byte loads (tiles of other waves left as zeros)
      const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
          a.partials + static_cast<int64_t>(mn) * a.splits * n_chunks * (C::BM * C::BN), 0, -1,
          kRsrcWord3);
      const uint32_t split_bytes = static_cast<uint32_t>(n_chunks * (C::BM * C::BN)) * 4u;
      auto load_part = [&](f32x16 (&dst)[TM][TN], uint32_t voff) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if (!mine(i, j)) {
#pragma unroll
                for (int c = 0; c < 4; ++c) dst[i][j][4 * q + c] = 0.0f;
                continue;
              }
              const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
                  pr, voff + ((i * TN + j) * 4 + q) * 1024, 0, kSystemCoherent);
#pragma unroll
              for (int c = 0; c < 4; ++c) dst[i][j][4 * q + c] = __int_as_float(v[c]);
            }
      };
      for (int tc = 0; tc < n_chunks; ++tc) {
        const uint32_t voff = static_cast<uint32_t>(tc * (C::BM * C::BN) + wmn * kPartFloats) * 4u +
                              static_cast<uint32_t>(lane) * 16u;
        f32x16 acc[TM][TN];
        load_part(acc, voff);
        for (int sp = 1; sp < a.splits; ++sp) {  // fixed summation order
          f32x16 part[TM][TN];
          load_part(part, voff + sp * split_bytes);
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
        }
        epilogue(acc, tc);
      }
    }
    if (tid == 0)  // ready for the next launch
      __hip_atomic_store(a.tickets + mn, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int WM, int WN, int TM, int TN, int KSPLIT, int NBUF, bool POOL, int MODE, int TAPS,
          bool PK>
int launch_cfg(const ConvArgs& a, hipStream_t stream) {
  if constexpr (NBUF == 0 && !PK) {
    return SNNK_EUNSUPPORTED;  // resident weights read packed spikes only
  } else if constexpr (!Cfg<WM, WN, TM, TN, KSPLIT, NBUF, PK>::kFits) {
    return SNNK_EUNSUPPORTED;  // this tile's ring does not fit LDS in this A format
  } else {
    using C = Cfg<WM, WN, TM, TN, KSPLIT, NBUF, PK>;
    if (C::kRes && (a.Cin % kKS != 0 || a.stages_per_split > C::kResStages))
      return SNNK_EUNSUPPORTED;
    const int64_t per_xcd = (static_cast<int64_t>(a.tiles_m) * a.tiles_n * a.splits + 7) / 8;
    if (per_xcd * 8 > 0x7FFFFFFFll) return SNNK_EUNSUPPORTED;
    // resident weights: the block's K stages of BN rows (at least the word
    // of the split-K ticket result)
    const unsigned dyn_lds =
        C::kRes ? static_cast<unsigned>(std::max(4, a.stages_per_split * C::BN * kRowBytes)) : 0u;
    hipLaunchKernelGGL((conv3x3_kernel<WM, WN, TM, TN, KSPLIT, NBUF, POOL, MODE, TAPS, PK>),
                       dim3(static_cast<unsigned>(per_xcd * 8)), dim3(C::kThreads), dyn_lds, stream, a);
    return launch_status();
  }
}

// tile configurations from this one on keep their weights resident (NBUF = 0)
constexpr int kFirstResCfg = 29;

struct Plan {
  int cfg, splits, stages_per_split, tiles_m, tiles_n;
  int64_t ticket_bytes, ws_bytes;
};

template <bool POOL, int MODE, int TAPS, bool PK>
int dispatch(const ConvArgs& a0, const Plan& p, void* workspace, hipStream_t s) {
  ConvArgs a = a0;
  a.tiles_m = p.tiles_m;
  a.tiles_n = p.tiles_n;
  a.div_tiles_m = make_fastdiv(static_cast<uint32_t>(std::max(1, p.tiles_m)));
  a.div_tiles_n = make_fastdiv(static_cast<uint32_t>(std::max(1, p.tiles_n)));
  a.splits = p.splits;
  a.stages_per_split = p.stages_per_split;
  // (resident-weight tiles: Cout-tile major, so that each XCD fills its
  // blocks' LDS from one or two weight slices held in its L2)
  a.n_major = p.splits == 1 && (a.w_bytes > a.x_bytes || p.cfg >= kFirstResCfg) ? 1 : 0;
  a.tickets = static_cast<unsigned int*>(workspace);
  a.partials = p.splits > 1
      ? reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + p.ticket_bytes) : nullptr;
  //                               WM WN TM TN KS NBUF           block tile, LDS
  switch (p.cfg) {
    case 0: return launch_cfg<2, 2, 2, 4, 1, 3, POOL, MODE, TAPS, PK>(a, s);   // 128 x 256, 144 KB
    case 1: return launch_cfg<4, 1, 2, 2, 1, 2, POOL, MODE, TAPS, PK>(a, s);   // 256 x 64, 80 KB
    case 2: return launch_cfg<2, 2, 2, 2, 1, 2, POOL, MODE, TAPS, PK>(a, s);   // 128 x 128, 64 KB
    case 3: return launch_cfg<2, 2, 1, 2, 1, 3, POOL, MODE, TAPS, PK>(a, s);   // 64 x 128, 72 KB
    case 4: return launch_cfg<1, 1, 1, 1, 4, 3, POOL, MODE, TAPS, PK>(a, s);   // 32 x 32 split-K 4, 96 KB
    case 5: return launch_cfg<1, 2, 1, 2, 2, 2, POOL, MODE, TAPS, PK>(a, s);   // 32 x 128 split-K 2, 80 KB
    case 6: return launch_cfg<1, 1, 1, 1, 8, 2, POOL, MODE, TAPS, PK>(a, s);   // 32 x 32 split-K 8, 128 KB
    case 7: return launch_cfg<1, 1, 1, 2, 4, 2, POOL, MODE, TAPS, PK>(a, s);   // 32 x 64 split-K 4, 96 KB
    case 8: return launch_cfg<1, 2, 1, 2, 4, 2, POOL, MODE, TAPS, PK>(a, s);   // 32 x 128 split-K 4, 160 KB
    case 9: return launch_cfg<2, 2, 2, 2, 2, 2, POOL, MODE, TAPS, PK>(a, s);   // 128 x 128 split-K 2, 128 KB
    case 10: return launch_cfg<4, 1, 1, 2, 1, 3, POOL, MODE, TAPS, PK>(a, s);  // 128 x 64, 72 KB
    case 11: return launch_cfg<2, 2, 2, 2, 1, 3, POOL, MODE, TAPS, PK>(a, s);  // 128 x 128, 96 KB
    case 12: return launch_cfg<4, 1, 1, 2, 1, 4, POOL, MODE, TAPS, PK>(a, s);  // 128 x 64, 96 KB
    case 13: return launch_cfg<1, 1, 1, 2, 2, 3, POOL, MODE, TAPS, PK>(a, s);  // 32 x 64 split-K 2, 72 KB
    case 14: return launch_cfg<4, 2, 2, 2, 1, 3, POOL, MODE, TAPS, PK>(a, s);  // 256 x 128, 144 KB
    case 15: return launch_cfg<2, 2, 2, 2, 1, 4, POOL, MODE, TAPS, PK>(a, s);  // 128 x 128, 128 KB
    case 16: return launch_cfg<2, 2, 1, 2, 1, 4, POOL, MODE, TAPS, PK>(a, s);  // 64 x 128, 96 KB
    case 17: return launch_cfg<4, 1, 1, 2, 1, 5, POOL, MODE, TAPS, PK>(a, s);  // 128 x 64, 120 KB
    case 18: return launch_cfg<1, 2, 1, 2, 2, 3, POOL, MODE, TAPS, PK>(a, s);  // 32 x 128 split-K 2, 120 KB
    // four-wave and two-wave blocks with 128 x 64 / 64 x 128 per wave (fewer
    // LDS fragment reads per MFMA than the 64 x 64 waves), and the 8-wave
    // 128 x 256 transpose of 14
    case 19: return launch_cfg<2, 2, 4, 2, 1, 3, POOL, MODE, TAPS, PK>(a, s);  // 256 x 128, 144 KB
    case 20: return launch_cfg<2, 2, 2, 4, 1, 3, POOL, MODE, TAPS, PK>(a, s);  // 128 x 256, 144 KB
    case 21: return launch_cfg<2, 4, 2, 2, 1, 3, POOL, MODE, TAPS, PK>(a, s);  // 128 x 256, 144 KB
    case 22: return launch_cfg<2, 1, 4, 2, 1, 2, POOL, MODE, TAPS, PK>(a, s);  // 256 x 64, 80 KB
    case 23: return launch_cfg<1, 2, 4, 2, 1, 2, POOL, MODE, TAPS, PK>(a, s);  // 128 x 128, 64 KB
    case 24: return launch_cfg<2, 1, 2, 4, 1, 2, POOL, MODE, TAPS, PK>(a, s);  // 128 x 128, 64 KB
    // deeper rings (4-5 stages) for the layers that stream their weights
    // from memory: more stages in flight per block hide the longer latency
    case 25: return launch_cfg<1, 1, 1, 1, 4, 5, POOL, MODE, TAPS, PK>(a, s);  // 32 x 32 split-K 4, 160 KB
    case 26: return launch_cfg<1, 1, 1, 2, 2, 5, POOL, MODE, TAPS, PK>(a, s);  // 32 x 64 split-K 2, 120 KB
    case 27: return launch_cfg<2, 2, 1, 2, 1, 5, POOL, MODE, TAPS, PK>(a, s);  // 64 x 128, 120 KB
    case 28: return launch_cfg<1, 2, 1, 2, 2, 4, POOL, MODE, TAPS, PK>(a, s);  // 32 x 128 split-K 2, 160 KB
    // resident weights (packed x only): all of K of the block's weight rows
    // in LDS, K up to 160 KB / (2 * BN)
    case 29: return launch_cfg<8, 1, 2, 2, 1, 0, POOL, MODE, TAPS, PK>(a, s);  // 512 x 64, K <= 1280
    case 30: return launch_cfg<4, 1, 2, 2, 1, 0, POOL, MODE, TAPS, PK>(a, s);  // 256 x 64, K <= 1280
    case 31: return launch_cfg<8, 1, 2, 1, 1, 0, POOL, MODE, TAPS, PK>(a, s);  // 512 x 32, K <= 2560
    case 32: return launch_cfg<4, 1, 2, 4, 1, 0, POOL, MODE, TAPS, PK>(a, s);  // 256 x 128, K <= 640
    case 33: return launch_cfg<4, 1, 2, 1, 1, 0, POOL, MODE, TAPS, PK>(a, s);  // 256 x 32, K <= 2560
    case 34: return launch_cfg<8, 1, 1, 2, 1, 0, POOL, MODE, TAPS, PK>(a, s);  // 256 x 64, K <= 1280
    // sixteen waves (four per SIMD), 32 rows each
    case 35: return launch_cfg<16, 1, 1, 2, 1, 0, POOL, MODE, TAPS, PK>(a, s);  // 512 x 64, K <= 1280
    case 36: return launch_cfg<16, 1, 1, 1, 1, 0, POOL, MODE, TAPS, PK>(a, s);  // 512 x 32, K <= 2560
    case 37: return launch_cfg<8, 1, 1, 1, 1, 0, POOL, MODE, TAPS, PK>(a, s);   // 256 x 32, K <= 2560
    // 128 weight columns per wave (each expanded spike fragment feeds four MFMAs)
    case 38: return launch_cfg<8, 1, 1, 4, 1, 0, POOL, MODE, TAPS, PK>(a, s);   // 256 x 128, K <= 640
    // 64-row ring tiles with K spread over 2-8 wave groups, for the layers
    // with few rows and long K (each weight byte re-read by half as many row
    // tiles as with 32-row tiles)
    case 39: return launch_cfg<2, 1, 1, 2, 4, 3, POOL, MODE, TAPS, PK>(a, s);   // 64 x 64 split-K 4
    case 40: return launch_cfg<2, 1, 1, 2, 8, 2, POOL, MODE, TAPS, PK>(a, s);   // 64 x 64 split-K 8
    case 41: return launch_cfg<2, 1, 1, 2, 2, 4, POOL, MODE, TAPS, PK>(a, s);   // 64 x 64 split-K 2
    // 64 x 32 with K over 4 wave groups: the FC layers over 128-224 rows,
    // each weight byte read by half as many row tiles as with 32-row tiles
    case 42: return launch_cfg<2, 1, 1, 1, 4, 3, POOL, MODE, TAPS, PK>(a, s);   // 64 x 32 split-K 4
    // 128 x 64 with K over 4 wave groups, 16 waves: the 4x4 layers at batch
    // 56 (3584 rows: 224 tiles, one round of blocks instead of 1.75 rounds
    // of 64 x 64 tiles)
    case 43: return launch_cfg<4, 1, 1, 2, 4, 3, POOL, MODE, TAPS, PK>(a, s);   // 128 x 64 split-K 4
    default: return SNNK_EINVAL;
  }
}

// Packed-input variants, instantiated in conv_packed.hip: the 3x3 conv
// with or without the 2x2 pool (taps = 9), the Linear with or without the
// OR of column groups of four (taps = 1), and the pre-activation Linear.
int dispatch_packed(const ConvArgs& a, const Plan& p, void* workspace, hipStream_t s, bool pool,
                    int taps, bool preact);

}  // namespace snnk
