// Fused conv3x3 (stride 1, pad 1) + folded-BN bias + multi-step LIF
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
#include <algorithm>
#include <mutex>

#include "conv_kernel.h"

namespace snnk {
namespace {

constexpr int kNumTiles = 44;
struct TileShape { int bm, bn; };
//                                   0          1         2          3         4        5
constexpr TileShape kTile[kNumTiles] = {{128, 256}, {256, 64}, {128, 128}, {64, 128}, {32, 32}, {32, 128},
//   6         7         8          9           10         11          12         13
    {32, 32}, {32, 64}, {32, 128}, {128, 128}, {128, 64}, {128, 128}, {128, 64}, {32, 64},
//   14          15          16         17         18          19          20          21
    {256, 128}, {128, 128}, {64, 128}, {128, 64}, {32, 128}, {256, 128}, {128, 256}, {128, 256},
//   22         23          24          25        26        27         28
    {256, 64}, {128, 128}, {128, 128}, {32, 32}, {32, 64}, {64, 128}, {32, 128},
//   29 - 38: resident weights, packed x only
    {512, 64}, {256, 64}, {512, 32}, {256, 128}, {256, 32}, {256, 64}, {512, 64}, {512, 32},
    {256, 32}, {256, 128},
//   39         40         41        42         43
    {64, 64}, {64, 64}, {64, 64}, {64, 32}, {128, 64}};

// Tile shape by problem size (rows = output rows of one 4-step chunk, K =
// 9*Cin or the Linear depth): big tiles while M fills 256 CUs, split-K wave
// groups as M shrinks and K grows.
int auto_cfg(const ConvArgs& a) {
  const int64_t rows = static_cast<int64_t>(a.n_quads) * 16;
  const int64_t K = static_cast<int64_t>(a.n_stages) * kKS;
  if (rows >= 65536) return 1;                                        // 256 x 64
  if (rows >= 32768) return a.Cout >= 256 ? 14 : (K <= 576 ? 3 : 9);
  if (rows >= 8192 && K <= 512) return a.Cout <= 512 ? 9 : 2;        // short K (SSA projections)
  if (rows >= 8192) return 3;                                         // 64 x 128
  if (rows >= 2048) return 18;                                        // 32 x 128 split-K 2
  if (rows >= 512) return 4;                                          // 32 x 32 split-K 4
  if (a.Cout <= 64) return 6;                                         // 32 x 32 split-K 8
  if (K <= 1024) return 7;                                            // 32 x 64 split-K 4
  return rows >= 128 ? 13 : 4;
}

// Tile shape and cross-block split when a workspace can be used, from a
// sweep of both over the VGG16 / SSA shapes: splitting pays for the
// weight-streaming small-M layers (FC, 4x4 with K = 4608).
void auto_cfg_split(const ConvArgs& a, int* cfg, int* splits) {
  const int64_t rows = static_cast<int64_t>(a.n_quads) * 16;
  const int64_t K = static_cast<int64_t>(a.n_stages) * kKS;
  *cfg = auto_cfg(a);
  *splits = 1;
  // Small M at modest Cout (the VGG layers at batch 1, from a sweep there):
  // 32x32 tiles for the most blocks, K spread over the wave groups and, for
  // the deep 4x4 and 2x2 layers, over 3 blocks per tile as well (L9 at
  // batch 1: 9.2 us against 14.2 us with 32x64 tiles and 2 splits).
  if (rows >= 16 && rows <= 1024 && a.Cout > 64 && a.Cout <= 512) {
    if (K <= 1152) { *cfg = 4; *splits = 1; }           // 32 x 32, 4 K groups
    else if (rows >= 256) { *cfg = 6; *splits = 1; }    // 32 x 32, 8 K groups
    else { *cfg = 4; *splits = 3; }
    return;
  }
  if (rows > 1024 && rows <= 8192 && a.Cout <= 64) { *cfg = 4; return; }  // 32x128 would idle half
  // M between the batch-32 and batch-56 VGG shapes (from a sweep at 56):
  // the 8x8 layers take 128x128 tiles (with 2 K groups past K = 2048), the
  // 4x4 layers 64x128 tiles (L9 at batch 56: 28.8 us against 52 us with the
  // batch-32 fallback of 32x128 tiles and no split)
  if (rows > 8192 && rows <= 16384 && a.Cout <= 512) { *cfg = K >= 2048 ? 9 : 11; return; }
  if (rows > 2048 && rows <= 4096 && a.Cout <= 1024) {
    if (K >= 4096) { *cfg = 3; *splits = 2; }                         // 64 x 128, 2 splits
    else *cfg = 16;                                                   // 64 x 128, 4 stages
    return;
  }
  if (rows > 2048 || rows < 16) return;
  if (rows > 512) {
    if (K >= 4096) { *cfg = 10; *splits = 4; }                        // 128 x 64, 4 splits
  } else if (rows > 128 && rows <= 256) {                             // FC layers at batch 56
    if (a.Cout <= 64) { *cfg = 4; *splits = 4; }                      // 32 x 32
    else if (K <= 512) { *cfg = 18; *splits = 1; }                    // 32 x 128, 2 K groups
    else if (K > 2048) { *cfg = 3; *splits = 3; }                     // 64 x 128, 3 splits
    else if (K > 1024 && a.Cout <= 2048) { *cfg = 13; *splits = 2; }  // 32 x 64
  } else if (rows <= 128) {
    if (a.Cout <= 64) { *cfg = 4; *splits = 4; }                      // 32 x 32
    else if (rows <= 32) { *cfg = 4; *splits = 1; }                   // FC layers at batch 1
    else if (K > 2048 || (K > 1024 && a.Cout > 2048)) { *cfg = 13; *splits = 2; }  // 32 x 64
    else if (K > 1024) { *cfg = 4; *splits = 1; }  // 32 x 32, 4 K groups: 2x2 maps as Linear
  }
}

// Workspace layout: a fixed ticket region (one counter per output tile,
// always at the same place so counters stay zero across calls of any shape)
// followed by the partial sums of the current call.
constexpr int64_t kMaxTickets = 65536;
constexpr int64_t kTicketBytes = kMaxTickets * 4;


// Tile shape and split for packed-spike input, from sweeps of every (tile,
// splits) pair over the VGG16 layers at batch 1, 32 and 56: with the A
// operand 16x smaller in LDS, taller tiles and more K groups pay where the
// bf16 rule picked small ones (VGG L4 at batch 32: 16.3 us with 128x128 tiles
// and 2 K groups against 22.2 with 256x128; L2 at batch 56: 27.8 us with
// 128x64 against 47.7 with 128x128).  Batch 1 keeps the bf16 rule.
bool auto_cfg_packed(const ConvArgs& a, bool taps9, int* cfg, int* splits) {
  const int64_t rows = static_cast<int64_t>(a.n_quads) * 16;
  const int64_t K = static_cast<int64_t>(a.n_stages) * kKS;
  const bool pool = a.Ho != a.H;
  *splits = 1;
  // Resident-weight tiles for the 3x3 layers with many rows, from sweeps at
  // batch 8, 32 and 56 (conv config at batch 32: 20.7 us against 23.5; VGG
  // L2-L7 20-24% faster).  Score: how well the tile count fills the 256 CUs
  // (tiles / whole waves of 256 blocks), weighted 0.55 for 32-column tiles,
  // whose waves expand each spike fragment for one MFMA instead of two (VGG
  // L2 at batch 56: 256x32 tiles fill 1.0 and take 42 us, 512x64 fill 0.875
  // and take 25); ties to 64 columns, then 512 rows, or 256 rows where two
  // blocks' weights fit a CU's LDS (VGG L2 at batch 56: 23.0 us with 256 x 64
  // tiles, two blocks per CU, against 24.6 with 512 x 64).  Below half a wave
  // of blocks, or below 8192 rows (batch 1), the streamed tiles are faster.
  if (taps9 && rows >= 8192 && a.Cin % kKS == 0) {
    struct Res { int cfg, bm, bn; };
    const bool two_per_cu = K * 64 * 2 * 2 <= kResBytes;
    const Res kRes[] = {two_per_cu ? Res{34, 256, 64} : Res{35, 512, 64},
                        two_per_cu ? Res{35, 512, 64} : Res{34, 256, 64},
                        {31, 512, 32}, {37, 256, 32}};
    int best = -1;
    double best_score = 0.0, best_fill = 0.0;
    for (const Res& r : kRes) {
      if (K * r.bn * 2 > kResBytes) continue;
      const int64_t tiles = ((a.n_quads + r.bm / 16 - 1) / (r.bm / 16)) *
                            ((a.Cout + r.bn - 1) / r.bn);
      const double fill = static_cast<double>(tiles) / (((tiles + 255) / 256) * 256);
      const double score = fill * (r.bn >= 64 ? 1.0 : 0.55);
      if (score > best_score + 1e-9) { best = r.cfg; best_score = score; best_fill = fill; }
    }
    if (best >= 0 && best_fill >= 0.5) { *cfg = best; return true; }
  }
  if (!taps9) {                                   // Linear (FC, dense 2x2 maps)
    // short-K projections over many rows (the SSA block's QKV: 8192 rows,
    // K = 384, 1152 columns: 17.8 us with 128 x 64 tiles, 21.9 with 128 x 128)
    if (rows >= 8192 && K <= 512) { *cfg = a.Cout > 512 ? 10 : 9; return true; }
    if (rows <= 64 || rows > 256) return false;
    // FC2 (K = 4096): 64x32 tiles with 4 K groups at batch 32 (12.2 us
    // against 14.3 with 32x32 tiles), 64x64 with 4 groups at batch 56 (14.9
    // against 17.4 with 64x32); the dense 2x2 layers (K = 2048) at batch 56:
    // 64x32 tiles, 4 groups, no split (8.4 us against 9.4 with 32x32); FC1
    // (K = 512, 4096 columns) at batch 56: 64x64 tiles, 2 groups (7.4
    // against 8.0)
    if (K >= 4096) { *cfg = rows <= 128 ? 42 : 39; return true; }
    if (K >= 2048) { if (rows <= 128) return false; *cfg = 42; return true; }
    if (K <= 512) { *cfg = rows <= 128 ? 4 : a.Cout > 512 ? 41 : 7; return true; }
    return false;
  }
  if (rows >= 65536) {                            // VGG L2 at batch 32 / 56
    if (a.Cout > 64) return false;
    *cfg = pool && rows >= 196608 ? 10 : 1;
    return true;
  }
  if (rows >= 32768) {                            // L3, L4
    // wider layers (the 128 -> 256 block at 16x16): 256 x 128 tiles, one
    // block per CU (21.6 us against 31.5 with the 2-group 128 x 128 tiles)
    if (a.Cout >= 256) *cfg = 14;
    else if (rows >= 49152) *cfg = pool ? 14 : 2;
    else *cfg = pool ? 9 : 10;
    return true;
  }
  if (rows >= 8192) {                             // L5 - L7
    if (a.Cout >= 512) *cfg = rows >= 12288 ? 14 : 9;
    else if (K <= 1152) *cfg = 10;
    else if (rows >= 12288) *cfg = 9;
    else *cfg = pool ? 5 : 12;
    return true;
  }
  if (rows >= 2048) {                             // L8 - L10
    if (K <= 1152) { *cfg = 4; return true; }
    // 64x64 tiles, K over 4 wave groups at batch 32 (2048 rows: L9 18.5 us
    // against 20.9 with 32x64 tiles): each weight byte is re-read by half as
    // many row tiles as with 32-row tiles.  At batch 56 (3584 rows) 128x64
    // tiles with 4 K groups and 16 waves, one round of 224 blocks (L9 23.3 us
    // against 26.1 with 64x64 tiles and 2 groups, L10 22.5 against 26.0)
    *cfg = rows <= 2048 ? 39 : 43;
    return true;
  }
  return false;
}

// packed_taps: 0 for bf16 x, else the kernel's taps (9: conv, 1: Linear)
// with packed x, which has its own plan rule
int make_plan(const ConvArgs& a, int tile_hint, int splits_hint, bool allow_split, Plan* p,
              int packed_taps = 0) {
  if (tile_hint >= kNumTiles || splits_hint < 0) return SNNK_EINVAL;
  int auto_splits = 1;
  if (tile_hint >= 0) p->cfg = tile_hint;
  else if (packed_taps != 0 && allow_split && splits_hint != 1 &&
           auto_cfg_packed(a, packed_taps == 9, &p->cfg, &auto_splits)) {
  } else if (allow_split && splits_hint != 1) auto_cfg_split(a, &p->cfg, &auto_splits);
  else p->cfg = auto_cfg(a);
  const TileShape ts = kTile[p->cfg];
  p->tiles_m = (a.n_quads + ts.bm / 16 - 1) / (ts.bm / 16);
  p->tiles_n = (a.Cout + ts.bn - 1) / ts.bn;
  const int64_t mn = static_cast<int64_t>(p->tiles_m) * p->tiles_n;
  int splits = 1;
  if (allow_split) {
    if (splits_hint > 0) splits = splits_hint;
    else if (tile_hint < 0) splits = auto_splits;
    else if (mn < 160) splits = static_cast<int>((256 + mn - 1) / mn);  // fill the GPU
    // at least 4 K stages per split; tile ids must fit the ticket region
    splits = std::max(1, std::min(splits, a.n_stages / 4));
    if (mn > kMaxTickets) splits = 1;
    // a tile's partial sums are addressed with 32-bit byte offsets
    const int64_t tile_part_bytes = static_cast<int64_t>((a.T + 3) / 4) * ts.bm * ts.bn * 4;
    if (splits * tile_part_bytes >= (int64_t{1} << 32)) splits = 1;
  }
  p->stages_per_split = (a.n_stages + splits - 1) / splits;
  p->splits = (a.n_stages + p->stages_per_split - 1) / p->stages_per_split;  // none empty
  p->ticket_bytes = 0;
  p->ws_bytes = 0;
  if (p->splits > 1) {
    const int64_t n_chunks = (a.T + 3) / 4;
    p->ticket_bytes = kTicketBytes;
    p->ws_bytes = p->ticket_bytes + mn * p->splits * n_chunks * ts.bm * ts.bn * 4;
  }
  return SNNK_OK;
}

// Validates a conv call and fills ConvArgs (no launch).
void set_row_divs(ConvArgs* a) {
  auto div = [](int d) { return make_fastdiv(static_cast<uint32_t>(std::max(d, 1))); };
  a->div_howo = div(a->Ho * a->Wo);
  a->div_wo = div(a->Wo);
  a->div_hw = div(a->H * a->W);
  a->div_w = div(a->W);
}

int conv_args(const uint16_t* x, const uint16_t* w, const float* bias, uint16_t* spikes_out,
              float* preact_out, int64_t T, int64_t B, int64_t H, int64_t W, int64_t Cin,
              int64_t Cout, int32_t pool, float decay, float in_scale, float v_threshold,
              float v_reset, int32_t soft_reset, bool check_ptrs, ConvArgs* out) {
  if (T < 0 || B < 0 || H < 0 || W < 0 || Cin <= 0 || Cout <= 0) return SNNK_EINVAL;
  const bool preact = preact_out != nullptr;
  if (check_ptrs) {
    if (x == nullptr || w == nullptr) return SNNK_EINVAL;
    if (!preact && spikes_out == nullptr) return SNNK_EINVAL;
  }
  if (preact && pool) return SNNK_EINVAL;
  if (Cin % 32 != 0 || Cout % 32 != 0) return SNNK_EUNSUPPORTED;
  if (pool && (H % 2 != 0 || W % 2 != 0)) return SNNK_EUNSUPPORTED;
  if (!pool && (B * H * W) % 4 != 0) return SNNK_EUNSUPPORTED;
  const int64_t step_in = B * H * W * Cin;
  const int64_t step_out = B * H * W * Cout;
  // byte offsets into x and w are 32-bit (buffer descriptors)
  if (T * step_in * 2 > kFar || T * step_out > (1ll << 40) || Cout * 9 * Cin * 2 > kFar)
    return SNNK_EUNSUPPORTED;
  if (check_ptrs && (!aligned(x, 16) || !aligned(w, 16))) return SNNK_EALIGN;
  ConvArgs a{};
  a.x = x; a.w = w; a.bias = bias; a.out = spikes_out; a.pre = preact_out;
  a.T = static_cast<int>(T); a.B = static_cast<int>(B);
  a.H = static_cast<int>(H); a.W = static_cast<int>(W);
  a.Cin = static_cast<int>(Cin); a.Cout = static_cast<int>(Cout);
  a.Ho = pool ? a.H / 2 : a.H;
  a.Wo = pool ? a.W / 2 : a.W;
  a.n_quads = pool ? a.B * a.Ho * a.Wo : a.B * a.H * a.W / 4;
  a.n_stages = static_cast<int>((9 * Cin + kKS - 1) / kKS);
  a.div_cin = make_fastdiv(static_cast<uint32_t>(Cin));
  set_row_divs(&a);
  a.x_tstride_b = static_cast<uint32_t>(step_in * 2);
  a.x_bytes = static_cast<uint32_t>(T * step_in * 2);
  a.w_bytes = static_cast<uint32_t>(Cout * 9 * Cin * 2);
  a.o_tstride = B * a.Ho * a.Wo * Cout;
  a.decay = decay; a.in_scale = in_scale; a.vth = v_threshold; a.v_reset = v_reset;
  a.soft_reset = soft_reset ? 1 : 0;
  *out = a;
  return SNNK_OK;
}

// Linear over the rows of [T][R][K]: the 1x1 case of the same kernel.
int linear_args(const uint16_t* x, const uint16_t* w, const float* bias, uint16_t* spikes_out,
                float* preact_out, int64_t T, int64_t R, int64_t K, int64_t N, float decay,
                float in_scale, float v_threshold, float v_reset, int32_t soft_reset,
                bool check_ptrs, ConvArgs* out, bool col_pool = false) {
  if (T < 0 || R < 0 || K <= 0 || N <= 0) return SNNK_EINVAL;
  if (check_ptrs) {
    if (x == nullptr || w == nullptr) return SNNK_EINVAL;
    if (preact_out == nullptr && spikes_out == nullptr) return SNNK_EINVAL;
  }
  if (K % 32 != 0 || N % 32 != 0 || R % 4 != 0) return SNNK_EUNSUPPORTED;
  if (T * R * K * 2 > kFar || N * K * 2 > kFar || T * R * N > (1ll << 40))
    return SNNK_EUNSUPPORTED;
  if (check_ptrs && (!aligned(x, 16) || !aligned(w, 16))) return SNNK_EALIGN;
  ConvArgs a{};
  a.x = x; a.w = w; a.bias = bias; a.out = spikes_out; a.pre = preact_out;
  a.T = static_cast<int>(T); a.B = 1; a.H = 1; a.W = static_cast<int>(R);
  a.Cin = static_cast<int>(K); a.Cout = static_cast<int>(N);
  a.Ho = 1; a.Wo = a.W;
  a.n_quads = static_cast<int>(R / 4);
  a.n_stages = static_cast<int>((K + kKS - 1) / kKS);
  a.div_cin = make_fastdiv(static_cast<uint32_t>(K));
  set_row_divs(&a);
  a.x_tstride_b = static_cast<uint32_t>(R * K * 2);
  a.x_bytes = static_cast<uint32_t>(T * R * K * 2);
  a.w_bytes = static_cast<uint32_t>(N * K * 2);
  a.o_tstride = col_pool ? R * (N / 4) : R * N;
  a.decay = decay; a.in_scale = in_scale; a.vth = v_threshold; a.v_reset = v_reset;
  a.soft_reset = soft_reset ? 1 : 0;
  *out = a;
  return SNNK_OK;
}

// Activation formats of the _act entry points: x read as packed words
// (x_bytes shrinks to the packed size; kernel offsets stay in bf16 bytes and
// are shifted down by 4 at the load), spikes written as packed words
// (o_tstride in words).  Packed words need 4-byte alignment.
int apply_act_formats(ConvArgs* a, const void* x, const void* out, int32_t x_fmt, int32_t out_fmt,
                      bool* packed_in) {
  if ((x_fmt != SNNK_ACT_BF16 && x_fmt != SNNK_ACT_BITS) ||
      (out_fmt != SNNK_ACT_BF16 && out_fmt != SNNK_ACT_BITS))
    return SNNK_EINVAL;
  if (x == nullptr || out == nullptr) return SNNK_EINVAL;
  *packed_in = x_fmt == SNNK_ACT_BITS;
  if (!aligned(x, *packed_in ? 4 : 16) || !aligned(out, out_fmt == SNNK_ACT_BITS ? 4 : 2))
    return SNNK_EALIGN;
  if (*packed_in) a->x_bytes /= 16;  // bf16 bytes are a multiple of 64
  if (out_fmt == SNNK_ACT_BITS) {
    a->bits_out = 1;
    a->o_tstride /= 32;
  }
  return SNNK_OK;
}

template <int TAPS>
int run(const ConvArgs& a, bool pool, int tile_hint, int splits, bool allow_split, void* ws,
        int64_t ws_bytes, hipStream_t s, bool mean = false, bool packed_in = false) {
  if (a.T == 0 || a.n_quads == 0) return SNNK_OK;
  Plan p;
  int st = make_plan(a, tile_hint, splits, allow_split, &p, packed_in ? TAPS : 0);
  if (st != SNNK_OK) return st;
  if (p.ws_bytes > 0 && (ws == nullptr || ws_bytes < p.ws_bytes)) return SNNK_EWORKSPACE;
  if (p.ws_bytes > 0 && !aligned(ws, 256)) return SNNK_EALIGN;
  if (packed_in || a.bits_out) {
    // LIF variants, and the pre-activation Linear on packed x; the
    // column-pooled Linear writes bf16 spikes
    const bool pre = a.pre != nullptr;
    if (mean || (pre && (a.bits_out || TAPS != 1 || pool)) || (TAPS == 1 && pool && a.bits_out))
      return SNNK_EUNSUPPORTED;
    if (packed_in) return dispatch_packed(a, p, ws, s, pool, TAPS, pre);
  }
  if constexpr (TAPS == 1) {
    if (mean) return dispatch<false, MODE_MEAN, 1, false>(a, p, ws, s);
    if (pool) return dispatch<true, MODE_LIF, 1, false>(a, p, ws, s);  // OR of column groups of 4
  }
  if (a.pre != nullptr) return dispatch<false, MODE_PREACT, TAPS, false>(a, p, ws, s);
  if (pool) return dispatch<true, MODE_LIF, TAPS, false>(a, p, ws, s);
  return dispatch<false, MODE_LIF, TAPS, false>(a, p, ws, s);
}

}  // namespace
}  // namespace snnk

using namespace snnk;

extern "C" int snnk_conv3x3_bn_lif(const uint16_t* x, const uint16_t* w, const float* bias,
                                   uint16_t* spikes_out, float* preact_out,
                                   int64_t T, int64_t B, int64_t H, int64_t W,
                                   int64_t Cin, int64_t Cout, int32_t pool,
                                   float decay, float in_scale, float v_threshold,
                                   float v_reset, int32_t soft_reset, int32_t tile_hint,
                                   void* stream) {
  ConvArgs a;
  if (T == 0 || B == 0 || H == 0 || W == 0) return (T < 0 || B < 0 || H < 0 || W < 0) ? SNNK_EINVAL : SNNK_OK;
  int st = conv_args(x, w, bias, spikes_out, preact_out, T, B, H, W, Cin, Cout, pool, decay,
                     in_scale, v_threshold, v_reset, soft_reset, true, &a);
  if (st != SNNK_OK) return st;
  return run<9>(a, pool != 0, tile_hint, 1, false, nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int snnk_conv3x3_bn_lif_ws(const uint16_t* x, const uint16_t* w, const float* bias,
                                      uint16_t* spikes_out, float* preact_out,
                                      int64_t T, int64_t B, int64_t H, int64_t W,
                                      int64_t Cin, int64_t Cout, int32_t pool,
                                      float decay, float in_scale, float v_threshold,
                                      float v_reset, int32_t soft_reset, int32_t tile_hint,
                                      int32_t splits, void* workspace, int64_t workspace_bytes,
                                      void* stream) {
  ConvArgs a;
  if (T == 0 || B == 0 || H == 0 || W == 0) return (T < 0 || B < 0 || H < 0 || W < 0) ? SNNK_EINVAL : SNNK_OK;
  int st = conv_args(x, w, bias, spikes_out, preact_out, T, B, H, W, Cin, Cout, pool, decay,
                     in_scale, v_threshold, v_reset, soft_reset, true, &a);
  if (st != SNNK_OK) return st;
  return run<9>(a, pool != 0, tile_hint, splits, true, workspace, workspace_bytes,
                static_cast<hipStream_t>(stream));
}

// ---- no-allocation variant: a fixed scratch region in device memory ---------
// The split-K tickets and partial sums of snnk_conv3x3_bn_lif_noalloc live in
// this array instead of a caller workspace.  Each GPU the library runs on
// holds its own copy for the life of the process.  In host code the name is
// only a stand-in: the per-device address comes from hipGetSymbolAddress.
constexpr int64_t kScratchBytes = int64_t{32} << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;

__global__ void zero_words_kernel(unsigned int* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Device address of `scratch` on the current device, resolved on the first
// call for that device; that call also clears the ticket region with a fill
// kernel on `s` (ordered before the caller's conv on the same stream).
int scratch_address(hipStream_t s, void** out) {
  static std::mutex mu;
  static void* addr[kMaxScratchDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return SNNK_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (p == nullptr || !aligned(p, 256)) return SNNK_EALIGN;
    constexpr int kWords = static_cast<int>(kTicketBytes / 4);
    hipLaunchKernelGGL(zero_words_kernel, dim3((kWords + 255) / 256), dim3(256), 0, s,
                       static_cast<unsigned int*>(p), kWords);
    const int st = launch_status();
    if (st != SNNK_OK) return st;
    addr[dev] = p;
  }
  *out = addr[dev];
  return SNNK_OK;
}

}  // namespace

extern "C" int snnk_conv3x3_bn_lif_noalloc(const uint16_t* x, const uint16_t* w,
                                           const float* bias, uint16_t* spikes_out,
                                           float* preact_out, int64_t T, int64_t B, int64_t H,
                                           int64_t W, int64_t Cin, int64_t Cout, int32_t pool,
                                           float decay, float in_scale, float v_threshold,
                                           float v_reset, int32_t soft_reset, int32_t tile_hint,
                                           int32_t splits, void* stream) {
  ConvArgs a;
  if (T == 0 || B == 0 || H == 0 || W == 0) return (T < 0 || B < 0 || H < 0 || W < 0) ? SNNK_EINVAL : SNNK_OK;
  int st = conv_args(x, w, bias, spikes_out, preact_out, T, B, H, W, Cin, Cout, pool, decay,
                     in_scale, v_threshold, v_reset, soft_reset, true, &a);
  if (st != SNNK_OK) return st;
  Plan p;
  st = make_plan(a, tile_hint, splits, true, &p);
  if (st != SNNK_OK) return st;
  if (p.ws_bytes > kScratchBytes) return SNNK_ESCRATCH;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if (p.ws_bytes > 0) {
    st = scratch_address(s, &ws);
    if (st != SNNK_OK) return st;
  }
  return run<9>(a, pool != 0, tile_hint, splits, true, ws, kScratchBytes, s);
}

extern "C" int64_t snnk_conv3x3_bn_lif_ws_size(int64_t T, int64_t B, int64_t H, int64_t W,
                                               int64_t Cin, int64_t Cout, int32_t pool,
                                               int32_t preact, int32_t tile_hint,
                                               int32_t splits) {
  if (T == 0 || B == 0 || H == 0 || W == 0) return (T < 0 || B < 0 || H < 0 || W < 0) ? SNNK_EINVAL : 0;
  ConvArgs a;
  float dummy = 0.0f;
  int st = conv_args(nullptr, nullptr, nullptr, nullptr, preact ? &dummy : nullptr, T, B, H, W,
                     Cin, Cout, pool, 0.f, 0.f, 0.f, 0.f, 0, false, &a);
  if (st != SNNK_OK) return st;
  Plan p;
  st = make_plan(a, tile_hint, splits, true, &p);
  return st != SNNK_OK ? st : p.ws_bytes;
}

extern "C" int snnk_linear_bias_lif(const uint16_t* x, const uint16_t* w, const float* bias,
                                    uint16_t* spikes_out, float* preact_out, int64_t T,
                                    int64_t R, int64_t K, int64_t N, float decay,
                                    float in_scale, float v_threshold, float v_reset,
                                    int32_t soft_reset, int32_t tile_hint, void* stream) {
  if (T == 0 || R == 0) return (T < 0 || R < 0) ? SNNK_EINVAL : SNNK_OK;
  ConvArgs a;
  int st = linear_args(x, w, bias, spikes_out, preact_out, T, R, K, N, decay, in_scale,
                       v_threshold, v_reset, soft_reset, true, &a);
  if (st != SNNK_OK) return st;
  return run<1>(a, false, tile_hint, 1, false, nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int snnk_linear_bias_lif_ws(const uint16_t* x, const uint16_t* w, const float* bias,
                                       uint16_t* spikes_out, float* preact_out, int64_t T,
                                       int64_t R, int64_t K, int64_t N, float decay,
                                       float in_scale, float v_threshold, float v_reset,
                                       int32_t soft_reset, int32_t tile_hint, int32_t splits,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
  if (T == 0 || R == 0) return (T < 0 || R < 0) ? SNNK_EINVAL : SNNK_OK;
  ConvArgs a;
  int st = linear_args(x, w, bias, spikes_out, preact_out, T, R, K, N, decay, in_scale,
                       v_threshold, v_reset, soft_reset, true, &a);
  if (st != SNNK_OK) return st;
  return run<1>(a, false, tile_hint, splits, true, workspace, workspace_bytes,
                static_cast<hipStream_t>(stream));
}

extern "C" int snnk_linear_bias_lif_pool4_ws(const uint16_t* x, const uint16_t* w,
                                             const float* bias, uint16_t* spikes_out, int64_t T,
                                             int64_t R, int64_t K, int64_t N, float decay,
                                             float in_scale, float v_threshold, float v_reset,
                                             int32_t soft_reset, int32_t tile_hint,
                                             int32_t splits, void* workspace,
                                             int64_t workspace_bytes, void* stream) {
  if (T == 0 || R == 0) return (T < 0 || R < 0) ? SNNK_EINVAL : SNNK_OK;
  if (spikes_out == nullptr) return SNNK_EINVAL;
  ConvArgs a;
  int st = linear_args(x, w, bias, spikes_out, nullptr, T, R, K, N, decay, in_scale,
                       v_threshold, v_reset, soft_reset, true, &a, true);
  if (st != SNNK_OK) return st;
  return run<1>(a, true, tile_hint, splits, true, workspace, workspace_bytes,
                static_cast<hipStream_t>(stream));
}

extern "C" int snnk_linear_mean_t(const uint16_t* x, const uint16_t* w, const float* bias,
                                  float* out, int64_t T, int64_t R, int64_t K, int64_t N,
                                  int32_t tile_hint, int32_t splits, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  if (T == 0 || R == 0) return (T < 0 || R < 0) ? SNNK_EINVAL : SNNK_OK;
  if (out == nullptr) return SNNK_EINVAL;
  ConvArgs a;
  int st = linear_args(x, w, bias, nullptr, out, T, R, K, N, 0.f, 0.f, 0.f, 0.f, 0, true, &a);
  if (st != SNNK_OK) return st;
  return run<1>(a, false, tile_hint, splits, true, workspace, workspace_bytes,
                static_cast<hipStream_t>(stream), true);
}

extern "C" int64_t snnk_linear_bias_lif_ws_size(int64_t T, int64_t R, int64_t K, int64_t N,
                                                int32_t preact, int32_t tile_hint,
                                                int32_t splits) {
  if (T == 0 || R == 0) return (T < 0 || R < 0) ? SNNK_EINVAL : 0;
  ConvArgs a;
  float dummy = 0.0f;
  int st = linear_args(nullptr, nullptr, nullptr, nullptr, preact ? &dummy : nullptr, T, R, K,
                       N, 0.f, 0.f, 0.f, 0.f, 0, false, &a);
  if (st != SNNK_OK) return st;
  Plan p;
  st = make_plan(a, tile_hint, splits, true, &p);
  return st != SNNK_OK ? st : p.ws_bytes;
}

extern "C" int snnk_conv3x3_bn_lif_act(const void* x, int32_t x_fmt, const uint16_t* w,
                                       const float* bias, void* spikes_out, int32_t out_fmt,
                                       int64_t T, int64_t B, int64_t H, int64_t W, int64_t Cin,
                                       int64_t Cout, int32_t pool, float decay, float in_scale,
                                       float v_threshold, float v_reset, int32_t soft_reset,
                                       int32_t tile_hint, int32_t splits, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  if (T == 0 || B == 0 || H == 0 || W == 0) return (T < 0 || B < 0 || H < 0 || W < 0) ? SNNK_EINVAL : SNNK_OK;
  if (w == nullptr || !aligned(w, 16)) return w == nullptr ? SNNK_EINVAL : SNNK_EALIGN;
  ConvArgs a;
  int st = conv_args(static_cast<const uint16_t*>(x), w, bias, static_cast<uint16_t*>(spikes_out),
                     nullptr, T, B, H, W, Cin, Cout, pool, decay, in_scale, v_threshold, v_reset,
                     soft_reset, false, &a);
  if (st != SNNK_OK) return st;
  bool packed_in = false;
  st = apply_act_formats(&a, x, spikes_out, x_fmt, out_fmt, &packed_in);
  if (st != SNNK_OK) return st;
  return run<9>(a, pool != 0, tile_hint, splits, true, workspace, workspace_bytes,
                static_cast<hipStream_t>(stream), false, packed_in);
}

extern "C" int snnk_linear_bias_lif_act(const void* x, int32_t x_fmt, const uint16_t* w,
                                        const float* bias, void* spikes_out, int32_t out_fmt,
                                        int64_t T, int64_t R, int64_t K, int64_t N,
                                        int32_t col_pool, float decay, float in_scale,
                                        float v_threshold, float v_reset, int32_t soft_reset,
                                        int32_t tile_hint, int32_t splits, void* workspace,
                                        int64_t workspace_bytes, void* stream) {
  if (T == 0 || R == 0) return (T < 0 || R < 0) ? SNNK_EINVAL : SNNK_OK;
  if (w == nullptr || !aligned(w, 16)) return w == nullptr ? SNNK_EINVAL : SNNK_EALIGN;
  ConvArgs a;
  int st = linear_args(static_cast<const uint16_t*>(x), w, bias,
                       static_cast<uint16_t*>(spikes_out), nullptr, T, R, K, N, decay, in_scale,
                       v_threshold, v_reset, soft_reset, false, &a, col_pool != 0);
  if (st != SNNK_OK) return st;
  bool packed_in = false;
  st = apply_act_formats(&a, x, spikes_out, x_fmt, out_fmt, &packed_in);
  if (st != SNNK_OK) return st;
  return run<1>(a, col_pool != 0, tile_hint, splits, true, workspace, workspace_bytes,
                static_cast<hipStream_t>(stream), false, packed_in);
}

extern "C" int snnk_linear_preact_act(const void* x, int32_t x_fmt, const uint16_t* w,
                                      const float* bias, float* out, int64_t T, int64_t R,
                                      int64_t K, int64_t N, int32_t tile_hint, int32_t splits,
                                      void* workspace, int64_t workspace_bytes, void* stream) {
  if (T == 0 || R == 0) return (T < 0 || R < 0) ? SNNK_EINVAL : SNNK_OK;
  if (w == nullptr || !aligned(w, 16)) return w == nullptr ? SNNK_EINVAL : SNNK_EALIGN;
  if (out == nullptr) return SNNK_EINVAL;
  ConvArgs a;
  int st = linear_args(static_cast<const uint16_t*>(x), w, bias, nullptr, out, T, R, K, N, 1.0f,
                       1.0f, 1.0f, 0.0f, 0, false, &a, false);
  if (st != SNNK_OK) return st;
  bool packed_in = false;
  st = apply_act_formats(&a, x, out, x_fmt, SNNK_ACT_BF16, &packed_in);
  if (st != SNNK_OK) return st;
  return run<1>(a, false, tile_hint, splits, true, workspace, workspace_bytes,
                static_cast<hipStream_t>(stream), false, packed_in);
}

extern "C" int64_t snnk_conv3x3_bn_lif_act_ws_size(int64_t T, int64_t B, int64_t H, int64_t W,
                                                   int64_t Cin, int64_t Cout, int32_t pool,
                                                   int32_t x_fmt, int32_t tile_hint,
                                                   int32_t splits) {
  if (T == 0 || B == 0 || H == 0 || W == 0) return (T < 0 || B < 0 || H < 0 || W < 0) ? SNNK_EINVAL : 0;
  if (x_fmt != SNNK_ACT_BF16 && x_fmt != SNNK_ACT_BITS) return SNNK_EINVAL;
  ConvArgs a;
  int st = conv_args(nullptr, nullptr, nullptr, nullptr, nullptr, T, B, H, W, Cin, Cout, pool,
                     0.f, 0.f, 0.f, 0.f, 0, false, &a);
  if (st != SNNK_OK) return st;
  Plan p;
  st = make_plan(a, tile_hint, splits, true, &p, x_fmt == SNNK_ACT_BITS ? 9 : 0);
  return st != SNNK_OK ? st : p.ws_bytes;
}

extern "C" int64_t snnk_linear_bias_lif_act_ws_size(int64_t T, int64_t R, int64_t K, int64_t N,
                                                    int32_t x_fmt, int32_t col_pool,
                                                    int32_t tile_hint, int32_t splits) {
  if (T == 0 || R == 0) return (T < 0 || R < 0) ? SNNK_EINVAL : 0;
  if (x_fmt != SNNK_ACT_BF16 && x_fmt != SNNK_ACT_BITS) return SNNK_EINVAL;
  ConvArgs a;
  int st = linear_args(nullptr, nullptr, nullptr, nullptr, nullptr, T, R, K, N, 0.f, 0.f, 0.f,
                       0.f, 0, false, &a, col_pool != 0);
  if (st != SNNK_OK) return st;
  Plan p;
  st = make_plan(a, tile_hint, splits, true, &p, x_fmt == SNNK_ACT_BITS ? 1 : 0);
  return st != SNNK_OK ? st : p.ws_bytes;
}
