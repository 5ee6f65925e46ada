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
// the KS wave groups take interleaved 32-wide K stages of the same output
// tile (group g: stages g, g+KS, ...; a group past the last stage loads
// zeros) and are summed through LDS before the epilogue (split-K for the
// small late layers).  Operand stages are double buffered in LDS.
#include "snnk_common.h"

namespace snnk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kKS = 32;           // K per stage
constexpr int kRow = kKS;         // LDS row pitch in bf16 (64 B, four 16-byte chunks)

// 16-byte chunk c of LDS row r is stored at chunk c ^ ((r >> 1) & 3): the
// staging writes (two rows x four chunks per 8 lanes) and the fragment reads
// (eight rows, one chunk per 8 lanes) then touch distinct bank groups.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 3); }

enum { MODE_LIF = 0, MODE_PREACT = 1 };

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
  int64_t x_tstride;  // B*H*W*Cin
  int64_t o_tstride;  // B*Ho*Wo*Cout
  float decay, in_scale, vth, v_reset;
  int soft_reset;
};

template <int WM, int WN, int TM, int TN, int KSPLIT, bool POOL, int MODE>
struct Cfg {
  static constexpr int kWaves = WM * WN * KSPLIT;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int BM = WM * TM * 32;
  static constexpr int BN = WN * TN * 32;
  static constexpr int kQuads = BM / 16;                    // quads per block
  static constexpr int kAChunks = KSPLIT * BM * (kKS / 8);  // 16-byte chunks
  static constexpr int kBChunks = KSPLIT * BN * (kKS / 8);
  static_assert(kAChunks % kThreads == 0, "A chunks must split evenly");
  static_assert(kBChunks % kThreads == 0, "B chunks must split evenly");
  static constexpr int kAPer = kAChunks / kThreads;
  static constexpr int kBPer = kBChunks / kThreads;
  static constexpr int kLdsA = KSPLIT * BM * kRow;  // bf16 elements per buffer
  static constexpr int kLdsB = KSPLIT * BN * kRow;
  static constexpr int kLdsBytes = 2 * (kLdsA + kLdsB) * 2;
  static constexpr int kRedBytes = (KSPLIT - 1) * WM * WN * TM * TN * 16 * 64 * 4;
  static constexpr int kSmem = kLdsBytes > kRedBytes ? kLdsBytes : kRedBytes;
};

__device__ __forceinline__ uint16_t spike_bf16(bool s) { return s ? 0x3F80u : 0u; }

// TAPS = 9: 3x3 conv, pad 1.  TAPS = 1: 1x1 conv, i.e. a Linear layer over
// the rows of [T][rows][Cin] (H = 1, W = rows).
template <int TAPS>
__device__ __forceinline__ int tap_dy(int tap) { return TAPS == 9 ? tap / 3 - 1 : 0; }
template <int TAPS>
__device__ __forceinline__ int tap_dx(int tap) { return TAPS == 9 ? tap % 3 - 1 : 0; }

template <int WM, int WN, int TM, int TN, int KSPLIT, bool POOL, int MODE, int TAPS>
__global__ __launch_bounds__(64 * WM * WN * KSPLIT)
void conv3x3_kernel(ConvArgs a) {
  using C = Cfg<WM, WN, TM, TN, KSPLIT, POOL, MODE>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[C::kSmem];
  uint16_t* ldsA = reinterpret_cast<uint16_t*>(smem);          // [2][KS][BM][kRow]
  uint16_t* ldsB = ldsA + 2 * C::kLdsA;                        // [2][KS][BN][kRow]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int kg = wave / (WM * WN);
  const int wmn = wave - kg * (WM * WN);
  const int wm = wmn / WN, wn = wmn - wm * WN;
  const int quad0 = blockIdx.x * C::kQuads;
  const int n0 = blockIdx.y * C::BN;
  const int HW = a.H * a.W;
  const int K = TAPS * a.Cin;

  // ---- per-thread A chunk geometry (fixed for the whole kernel) ----------
  // chunk c -> (group, row, 16-byte part); row -> (quad, pixel q, step t)
  int a_off[C::kAPer];      // element offset of (b, y, x, part*8) in one step
  int a_t[C::kAPer];        // step within the chunk of 4
  uint32_t a_ok[C::kAPer];  // bit tap: source pixel inside the image; bit 9: row valid
  int a_kg[C::kAPer];
  int a_lds[C::kAPer];      // LDS element offset inside a buffer
#pragma unroll
  for (int i = 0; i < C::kAPer; ++i) {
    const int c = tid + i * C::kThreads;
    const int g = c / (C::BM * 4);
    const int rem = c - g * (C::BM * 4);
    const int r = rem >> 2, part = rem & 3;
    const int rr = r & 31;
    const int q = rr >> 3, gr = (rr >> 2) & 1, t = rr & 3;
    const int quad = quad0 + (r >> 5) * 2 + gr;
    int b = 0, y = 0, xx = 0;
    const bool row_ok = quad < a.n_quads;
    if (row_ok) {
      if constexpr (POOL) {
        const int howo = a.Ho * a.Wo;
        b = quad / howo;
        const int r2 = quad - b * howo;
        const int py = r2 / a.Wo, px = r2 - py * a.Wo;
        y = 2 * py + (q >> 1);
        xx = 2 * px + (q & 1);
      } else {
        const int p = quad * 4 + q;
        b = p / HW;
        const int r2 = p - b * HW;
        y = r2 / a.W;
        xx = r2 - y * a.W;
      }
    }
    uint32_t ok = row_ok ? (1u << 9) : 0u;
#pragma unroll
    for (int tap = 0; tap < TAPS; ++tap) {
      const int ys = y + tap_dy<TAPS>(tap), xs = xx + tap_dx<TAPS>(tap);
      if (row_ok && ys >= 0 && ys < a.H && xs >= 0 && xs < a.W) ok |= 1u << tap;
    }
    a_off[i] = ((b * a.H + y) * a.W + xx) * a.Cin + part * 8;
    a_t[i] = t;
    a_ok[i] = ok;
    a_kg[i] = g;
    a_lds[i] = (g * C::BM + r) * kRow + swz(r, part) * 8;
  }
  int b_off[C::kBPer], b_kg[C::kBPer], b_lds[C::kBPer];
  bool b_ok[C::kBPer];
#pragma unroll
  for (int i = 0; i < C::kBPer; ++i) {
    const int c = tid + i * C::kThreads;
    const int g = c / (C::BN * 4);
    const int rem = c - g * (C::BN * 4);
    const int n = rem >> 2, part = rem & 3;
    b_ok[i] = n0 + n < a.Cout;
    b_off[i] = (b_ok[i] ? (n0 + n) : 0) * K + part * 8;
    b_kg[i] = g;
    b_lds[i] = (g * C::BN + n) * kRow + swz(n, part) * 8;
  }

  const int n_stages_g = (a.n_stages + KSPLIT - 1) / KSPLIT;
  const int n_chunks = (a.T + 3) / 4;

  // membrane state of the epilogue waves: [TM][TN][4 pixels]
  float v[TM][TN][4];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[i][j][q] = 0.0f;

  const int g_lane = lane >> 5, r_lane = lane & 31;
  float bias_n[TN];
  bool col_ok[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + (wn * TN + j) * 32 + r_lane;
    col_ok[j] = n < a.Cout;
    bias_n[j] = (a.bias && col_ok[j]) ? a.bias[n] : 0.0f;
  }

  for (int tc = 0; tc < n_chunks; ++tc) {
    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    u32x4 ra[C::kAPer], rb[C::kBPer];
    auto gload = [&](int s) {
#pragma unroll
      for (int i = 0; i < C::kAPer; ++i) {
        // a group whose interleaved stage runs past K loads zeros
        const int sg = s * KSPLIT + a_kg[i];
        const int k0 = (sg < a.n_stages ? sg : 0) * kKS;
        const int tap = TAPS == 9 ? static_cast<int>(fdiv(static_cast<uint32_t>(k0), a.div_cin)) : 0;
        const int cin0 = k0 - tap * a.Cin;
        const int tg = tc * 4 + a_t[i];
        u32x4 z = {0u, 0u, 0u, 0u};
        if (((a_ok[i] >> tap) & 1u) && (a_ok[i] >> 9) && tg < a.T && sg < a.n_stages) {
          const int dy = tap_dy<TAPS>(tap), dx = tap_dx<TAPS>(tap);
          const int64_t off = static_cast<int64_t>(tg) * a.x_tstride + a_off[i] +
                              (dy * a.W + dx) * a.Cin + cin0;
          z = *reinterpret_cast<const u32x4*>(a.x + off);
        }
        ra[i] = z;
      }
#pragma unroll
      for (int i = 0; i < C::kBPer; ++i) {
        const int sg = s * KSPLIT + b_kg[i];
        u32x4 z = {0u, 0u, 0u, 0u};
        if (b_ok[i] && sg < a.n_stages)
          z = *reinterpret_cast<const u32x4*>(a.w + b_off[i] + sg * kKS);
        rb[i] = z;
      }
    };
    auto lstore = [&](int buf) {
#pragma unroll
      for (int i = 0; i < C::kAPer; ++i)
        *reinterpret_cast<u32x4*>(ldsA + buf * C::kLdsA + a_lds[i]) = ra[i];
#pragma unroll
      for (int i = 0; i < C::kBPer; ++i)
        *reinterpret_cast<u32x4*>(ldsB + buf * C::kLdsB + b_lds[i]) = rb[i];
    };

    gload(0);
    lstore(0);
    __syncthreads();
    for (int s = 0; s < n_stages_g; ++s) {
      const int buf = s & 1;
      if (s + 1 < n_stages_g) gload(s + 1);
      const uint16_t* sa = ldsA + buf * C::kLdsA + (kg * C::BM + wm * TM * 32 + r_lane) * kRow;
      const uint16_t* sb = ldsB + buf * C::kLdsB + (kg * C::BN + wn * TN * 32 + r_lane) * kRow;
#pragma unroll
      for (int kk = 0; kk < kKS / 16; ++kk) {
        // tile rows start at multiples of 32, so the swizzle depends on r_lane only
        const int ch = swz(r_lane, kk * 2 + g_lane) * 8;
        bf16x8 fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          fa[i] = *reinterpret_cast<const bf16x8*>(sa + i * 32 * kRow + ch);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          fb[j] = *reinterpret_cast<const bf16x8*>(sb + j * 32 * kRow + ch);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
      }
      if (s + 1 < n_stages_g) lstore(buf ^ 1);
      __syncthreads();
    }

    // ---- split-K reduction through LDS ----------------------------------
    if constexpr (KSPLIT > 1) {
      float* red = reinterpret_cast<float*>(smem);
      if (kg > 0) {
        float* dst = red + ((kg - 1) * WM * WN + wmn) * TM * TN * 16 * 64;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) dst[((i * TN + j) * 16 + e) * 64 + lane] = acc[i][j][e];
      }
      __syncthreads();
      if (kg == 0) {
#pragma unroll
        for (int gg = 1; gg < KSPLIT; ++gg) {
          const float* src = red + ((gg - 1) * WM * WN + wmn) * TM * TN * 16 * 64;
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
              for (int e = 0; e < 16; ++e) acc[i][j][e] += src[((i * TN + j) * 16 + e) * 64 + lane];
        }
      }
      __syncthreads();
    }

    // ---- epilogue: bias + LIF over the 4 steps (+ 2x2 OR) -------------------
    if (kg == 0) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int quad = quad0 + (wm * TM + i) * 2 + g_lane;
        if (quad >= a.n_quads) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (!col_ok[j]) continue;
          const int n = n0 + (wn * TN + j) * 32 + r_lane;
          if constexpr (MODE == MODE_PREACT) {
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
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int tg = tc * 4 + t;
              if (tg >= a.T) break;
              bool any = false;
              bool sp[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const float u = __fadd_rn(acc[i][j][q * 4 + t], bias_n[j]);
                const float h = __fadd_rn(__fmul_rn(a.decay, v[i][j][q]), __fmul_rn(a.in_scale, u));
                const bool s = h >= a.vth;
                v[i][j][q] = s ? (a.soft_reset ? __fsub_rn(h, a.vth) : a.v_reset) : h;
                sp[q] = s;
                any = any || s;
              }
              uint16_t* o = a.out + static_cast<int64_t>(tg) * a.o_tstride;
              if constexpr (POOL) {
                o[static_cast<int64_t>(quad) * a.Cout + n] = spike_bf16(any);
              } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                  o[(static_cast<int64_t>(quad) * 4 + q) * a.Cout + n] = spike_bf16(sp[q]);
              }
            }
          }
        }
      }
    }
  }
}

template <int WM, int WN, int TM, int TN, int KSPLIT, bool POOL, int MODE, int TAPS>
int launch_cfg(const ConvArgs& a, hipStream_t stream) {
  using C = Cfg<WM, WN, TM, TN, KSPLIT, POOL, MODE>;
  const int gx = (a.n_quads + C::kQuads - 1) / C::kQuads;
  const int gy = (a.Cout + C::BN - 1) / C::BN;
  hipLaunchKernelGGL((conv3x3_kernel<WM, WN, TM, TN, KSPLIT, POOL, MODE, TAPS>), dim3(gx, gy),
                     dim3(C::kThreads), 0, stream, a);
  return launch_status();
}

// Tile shape by problem size (rows = output rows of one 4-step chunk, K =
// 9*Cin or the Linear depth), from a sweep of every config over the VGG16 and
// SSA layer shapes on MI355X: big tiles while M fills 256 CUs, split-K wave
// groups as M shrinks and K grows.
template <bool POOL, int MODE, int TAPS>
int dispatch(const ConvArgs& a, int tile_hint, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(a.n_quads) * 16;  // per T-chunk
  const int64_t K = static_cast<int64_t>(a.n_stages) * kKS;
  int cfg = tile_hint;
  if (cfg < 0) {
    if (rows >= 65536) cfg = 10;                       // 128 x 64
    else if (rows >= 32768) cfg = a.Cout >= 256 ? 2 : 9;  // 128 x 128 (split-K 2)
    else if (rows >= 8192) cfg = K <= 512 ? 10 : 8;    // 128 x 64 / 32 x 128 split-K 4
    else if (rows >= 2048) cfg = K <= 2304 ? 8 : 7;    // 32 x 128 / 32 x 64, split-K 4
    else if (rows >= 512 || a.Cout <= 64) cfg = 11;   // 32 x 32, split-K 16
    else cfg = K <= 1024 ? 4 : 6;                      // 32 x 32, split-K 4 / 8
  }
  switch (cfg) {
    case 0: return launch_cfg<2, 2, 2, 4, 1, POOL, MODE, TAPS>(a, s);
    case 1: return launch_cfg<4, 1, 2, 2, 1, POOL, MODE, TAPS>(a, s);
    case 2: return launch_cfg<2, 2, 2, 2, 1, POOL, MODE, TAPS>(a, s);
    case 3: return launch_cfg<2, 2, 1, 2, 1, POOL, MODE, TAPS>(a, s);
    case 4: return launch_cfg<1, 1, 1, 1, 4, POOL, MODE, TAPS>(a, s);
    case 5: return launch_cfg<1, 2, 1, 2, 2, POOL, MODE, TAPS>(a, s);
    case 6: return launch_cfg<1, 1, 1, 1, 8, POOL, MODE, TAPS>(a, s);   // 32 x 32, split-K 8
    case 7: return launch_cfg<1, 1, 1, 2, 4, POOL, MODE, TAPS>(a, s);   // 32 x 64, split-K 4
    case 8: return launch_cfg<1, 2, 1, 2, 4, POOL, MODE, TAPS>(a, s);   // 32 x 128, split-K 4
    case 9: return launch_cfg<2, 2, 2, 2, 2, POOL, MODE, TAPS>(a, s);   // 128 x 128, split-K 2
    case 10: return launch_cfg<4, 1, 1, 2, 1, POOL, MODE, TAPS>(a, s);  // 128 x 64
    case 11: return launch_cfg<1, 1, 1, 1, 16, POOL, MODE, TAPS>(a, s); // 32 x 32, split-K 16
    default: return SNNK_EINVAL;
  }
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
  if (T < 0 || B < 0 || H < 0 || W < 0 || Cin <= 0 || Cout <= 0) return SNNK_EINVAL;
  if (T == 0 || B == 0 || H == 0 || W == 0) return SNNK_OK;
  if (x == nullptr || w == nullptr) return SNNK_EINVAL;
  const bool preact = preact_out != nullptr;
  if (!preact && spikes_out == nullptr) return SNNK_EINVAL;
  if (preact && pool) return SNNK_EINVAL;
  if (Cin % kKS != 0 || Cout % 32 != 0) return SNNK_EUNSUPPORTED;
  if (pool && (H % 2 != 0 || W % 2 != 0)) return SNNK_EUNSUPPORTED;
  if (!pool && (B * H * W) % 4 != 0) return SNNK_EUNSUPPORTED;
  const int64_t step_in = B * H * W * Cin;
  const int64_t step_out = B * H * W * Cout;
  if (T * step_in > 0x7FFFFFFFll || T * step_out > (1ll << 40) || 9 * Cin > 0x7FFFFFFF ||
      B * H * W * Cin > 0x7FFFFFFFll || Cout * 9 * Cin > 0x7FFFFFFFll)
    return SNNK_EUNSUPPORTED;
  if (!aligned(x, 16) || !aligned(w, 16)) return SNNK_EALIGN;

  ConvArgs a{};
  a.x = x; a.w = w; a.bias = bias; a.out = spikes_out; a.pre = preact_out;
  a.T = static_cast<int>(T); a.B = static_cast<int>(B);
  a.H = static_cast<int>(H); a.W = static_cast<int>(W);
  a.Cin = static_cast<int>(Cin); a.Cout = static_cast<int>(Cout);
  a.Ho = pool ? a.H / 2 : a.H;
  a.Wo = pool ? a.W / 2 : a.W;
  a.n_quads = pool ? a.B * a.Ho * a.Wo : a.B * a.H * a.W / 4;
  a.n_stages = static_cast<int>(9 * Cin / kKS);
  a.div_cin = make_fastdiv(static_cast<uint32_t>(Cin));
  a.x_tstride = step_in;
  a.o_tstride = B * a.Ho * a.Wo * Cout;
  a.decay = decay; a.in_scale = in_scale; a.vth = v_threshold; a.v_reset = v_reset;
  a.soft_reset = soft_reset ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (preact) return dispatch<false, MODE_PREACT, 9>(a, tile_hint, s);
  if (pool) return dispatch<true, MODE_LIF, 9>(a, tile_hint, s);
  return dispatch<false, MODE_LIF, 9>(a, tile_hint, s);
}

// Linear + bias + LIF over T: x [T][R][K] bf16 rows, w [N][K] bf16 (the
// nn.Linear weight layout), one 1x1-conv pass of the same kernel.
extern "C" int snnk_linear_bias_lif(const uint16_t* x, const uint16_t* w, const float* bias,
                                    uint16_t* spikes_out, float* preact_out, int64_t T,
                                    int64_t R, int64_t K, int64_t N, float decay,
                                    float in_scale, float v_threshold, float v_reset,
                                    int32_t soft_reset, int32_t tile_hint, void* stream) {
  if (T < 0 || R < 0 || K <= 0 || N <= 0) return SNNK_EINVAL;
  if (T == 0 || R == 0) return SNNK_OK;
  if (x == nullptr || w == nullptr) return SNNK_EINVAL;
  const bool preact = preact_out != nullptr;
  if (!preact && spikes_out == nullptr) return SNNK_EINVAL;
  if (K % kKS != 0 || N % 32 != 0 || R % 4 != 0) return SNNK_EUNSUPPORTED;
  if (T * R * K > 0x7FFFFFFFll || R * K > 0x7FFFFFFFll || N * K > 0x7FFFFFFFll ||
      T * R * N > (1ll << 40))
    return SNNK_EUNSUPPORTED;
  if (!aligned(x, 16) || !aligned(w, 16)) return SNNK_EALIGN;
  ConvArgs a{};
  a.x = x; a.w = w; a.bias = bias; a.out = spikes_out; a.pre = preact_out;
  a.T = static_cast<int>(T); a.B = 1; a.H = 1; a.W = static_cast<int>(R);
  a.Cin = static_cast<int>(K); a.Cout = static_cast<int>(N);
  a.Ho = 1; a.Wo = a.W;
  a.n_quads = static_cast<int>(R / 4);
  a.n_stages = static_cast<int>(K / kKS);
  a.div_cin = make_fastdiv(static_cast<uint32_t>(K));
  a.x_tstride = R * K;
  a.o_tstride = R * N;
  a.decay = decay; a.in_scale = in_scale; a.vth = v_threshold; a.v_reset = v_reset;
  a.soft_reset = soft_reset ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (preact) return dispatch<false, MODE_PREACT, 1>(a, tile_hint, s);
  return dispatch<false, MODE_LIF, 1>(a, tile_hint, s);
}
