// Multi-step IF/LIF neuron for gfx950.
//
// One thread owns VEC consecutive neurons (16 bytes of input per step) and
// keeps their membrane state in VGPRs for the whole time loop.  The time loop
// is processed in chunks of 4 steps: the loads of all 4 steps (and of the
// residual) are issued before the dependent neuron arithmetic, so every lane
// has 4 x 16 B in flight.  Step order and rounding follow the reference
// recurrence (snn_compiler/kernels/fused.py:101-114,429-441 and the naive
// restatement at snn_compiler/kernels/neurons.py:493-500): every product and
// sum is rounded separately (__fmul_rn / __fadd_rn keep the compiler from
// contracting them into an FMA).
#include <type_traits>

#include "snnk_common.h"

namespace snnk {
namespace {

constexpr int kBlock = 256;
constexpr int kTChunk = 4;

struct LifArgs {
  const void* x;
  const float* bias;
  const void* residual;
  const float* vth;
  const float* v_init;
  float* v_out;
  void* spikes;
  float* count_out;
  int64_t T, NCL;
  uint32_t C;
  FastDiv div_hw;   // NCHW channel: (i / HW) % C
  FastDiv div_c;    // modulo C
  uint64_t HW64, C64;
  int32_t thr_mode, channel_last, soft_reset, use_div32;
  float vth_scalar, decay, in_scale, v_reset;
};

struct BF16 { typedef uint16_t raw; };
struct F16 { typedef uint16_t raw; };
struct F32 { typedef float raw; };

template <typename Tag> __device__ __forceinline__ float to_f32(typename Tag::raw v);
template <> __device__ __forceinline__ float to_f32<F32>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<BF16>(uint16_t v) { return bf16_to_f32(v); }
template <> __device__ __forceinline__ float to_f32<F16>(uint16_t v) { return f16_to_f32(v); }

template <typename Tag> __device__ __forceinline__ typename Tag::raw spike_val(bool s);
template <> __device__ __forceinline__ float spike_val<F32>(bool s) { return s ? 1.0f : 0.0f; }
template <> __device__ __forceinline__ uint16_t spike_val<BF16>(bool s) { return s ? 0x3F80u : 0u; }
template <> __device__ __forceinline__ uint16_t spike_val<F16>(bool s) { return s ? 0x3C00u : 0u; }

// VEC raw elements packed in one 16-byte (or smaller) register tuple.
template <typename Raw, int VEC>
struct Pack {
  Raw v[VEC];
};

template <typename Raw, int VEC>
__device__ __forceinline__ Pack<Raw, VEC> load_pack(const Raw* p) {
  Pack<Raw, VEC> r;
  if constexpr (sizeof(Raw) * VEC == 16) {
    u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    __builtin_memcpy(&r, &w, 16);
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) r.v[j] = p[j];
  }
  return r;
}

template <typename Raw, int VEC>
__device__ __forceinline__ void store_pack(Raw* p, const Pack<Raw, VEC>& r) {
  if constexpr (sizeof(Raw) * VEC == 16) {
    u32x4 w;
    __builtin_memcpy(&w, &r, 16);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
  } else if constexpr (sizeof(Raw) * VEC == 8) {
    u32x2 w;
    __builtin_memcpy(&w, &r, 8);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(p));
  } else if constexpr (sizeof(Raw) * VEC == 4) {
    uint32_t w;
    __builtin_memcpy(&w, &r, 4);
    __builtin_nontemporal_store(w, reinterpret_cast<uint32_t*>(p));
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) p[j] = r.v[j];
  }
}

// VEC floats of a per-neuron side buffer (v_init, v_out, count, threshold);
// VEC % 4 == 0 implies the buffer was checked for 16-byte alignment.
template <int VEC>
__device__ __forceinline__ void load_f32s(const float* p, float* out) {
  if constexpr (VEC % 4 == 0) {
#pragma unroll
    for (int j = 0; j < VEC; j += 4) {
      f32x4 w = *reinterpret_cast<const f32x4*>(p + j);
      out[j] = w.x; out[j + 1] = w.y; out[j + 2] = w.z; out[j + 3] = w.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) out[j] = p[j];
  }
}

template <int VEC>
__device__ __forceinline__ void store_f32s(float* p, const float* in) {
  if constexpr (VEC % 4 == 0) {
#pragma unroll
    for (int j = 0; j < VEC; j += 4) {
      f32x4 w = {in[j], in[j + 1], in[j + 2], in[j + 3]};
      __builtin_nontemporal_store(w, reinterpret_cast<f32x4*>(p + j));
    }
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) p[j] = in[j];
  }
}

__device__ __forceinline__ uint32_t channel_of(const LifArgs& a, uint64_t i) {
  if (a.use_div32) {
    uint32_t i32 = static_cast<uint32_t>(i);
    uint32_t q = a.channel_last ? i32 : fdiv(i32, a.div_hw);
    return q - fdiv(q, a.div_c) * a.C;
  }
  uint64_t q = a.channel_last ? i : i / a.HW64;
  return static_cast<uint32_t>(q % a.C64);
}

// v of another lane of the same 16-lane row (DPP control CTRL)
template <int CTRL>
__device__ __forceinline__ uint32_t lane_dpp(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// Tag: input element type; SPK: 0 = spikes in the input type, 1 = uint8,
// 2 = bf16, 3 = packed bits (a lane's VEC spike bits are OR-combined across
// the 32/VEC lanes of one 32-neuron word by DPP lane exchanges; NCL % 32 == 0 makes
// every word's lanes all active or all retired);
// VEC: neurons per thread (VEC == 1 is the unaligned / ragged fallback).
template <typename Tag, int SPK, int VEC, bool HAS_RES>
__global__ __launch_bounds__(kBlock) void lif_kernel(LifArgs a) {
  typedef typename Tag::raw Raw;
  typedef typename std::conditional<
      SPK == 0, Raw, typename std::conditional<SPK == 1, uint8_t, uint16_t>::type>::type SRaw;
  constexpr int kLanesPerWord = 32 / VEC;
  const uint64_t i0 =
      (static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x) * VEC;
  if (i0 >= static_cast<uint64_t>(a.NCL)) return;  // NCL % VEC == 0 when VEC > 1

  float v[VEC], thr[VEC], b[VEC], cnt[VEC];
  const bool need_c = (a.bias != nullptr) || (a.thr_mode == SNNK_THR_PER_CHANNEL);
  if (a.thr_mode == SNNK_THR_PER_NEURON) load_f32s<VEC>(a.vth + i0, thr);
  if (a.v_init) load_f32s<VEC>(a.v_init + i0, v);
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    uint32_t c = need_c ? channel_of(a, i0 + j) : 0u;
    b[j] = a.bias ? a.bias[c] : 0.0f;
    if (a.thr_mode == SNNK_THR_SCALAR) thr[j] = a.vth_scalar;
    else if (a.thr_mode == SNNK_THR_PER_CHANNEL) thr[j] = a.vth[c];
    if (!a.v_init) v[j] = 0.0f;
    cnt[j] = 0.0f;
  }
  const bool has_bias = a.bias != nullptr;
  const Raw* x = static_cast<const Raw*>(a.x);
  const Raw* r = static_cast<const Raw*>(a.residual);
  SRaw* s_out = static_cast<SRaw*>(a.spikes);
  const uint64_t ncl = static_cast<uint64_t>(a.NCL);

  for (int64_t t0 = 0; t0 < a.T; t0 += kTChunk) {
    Pack<Raw, VEC> xs[kTChunk], rs[kTChunk];
#pragma unroll
    for (int k = 0; k < kTChunk; ++k) {
      if (t0 + k < a.T) {
        const uint64_t off = static_cast<uint64_t>(t0 + k) * ncl + i0;
        xs[k] = load_pack<Raw, VEC>(x + off);
        if constexpr (HAS_RES) rs[k] = load_pack<Raw, VEC>(r + off);
      }
    }
#pragma unroll
    for (int k = 0; k < kTChunk; ++k) {
      if (t0 + k < a.T) {
        Pack<SRaw, VEC> so;
        uint32_t nib = 0;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          float u = to_f32<Tag>(xs[k].v[j]);
          if (has_bias) u = __fadd_rn(u, b[j]);
          if constexpr (HAS_RES) u = __fadd_rn(u, to_f32<Tag>(rs[k].v[j]));
          float h = __fadd_rn(__fmul_rn(a.decay, v[j]), __fmul_rn(a.in_scale, u));
          bool s = h >= thr[j];
          v[j] = s ? (a.soft_reset ? __fsub_rn(h, thr[j]) : a.v_reset) : h;
          cnt[j] += s ? 1.0f : 0.0f;
          if constexpr (SPK == 0) so.v[j] = spike_val<Tag>(s);
          else if constexpr (SPK == 1) so.v[j] = s ? 1 : 0;
          else if constexpr (SPK == 2) so.v[j] = s ? 0x3F80u : 0u;
          else nib |= (s ? 1u : 0u) << j;
        }
        if constexpr (SPK == 3) {
          const int lane = threadIdx.x & 63;
          uint32_t w = nib << (VEC * (lane % kLanesPerWord));
          // OR over the word's lanes: DPP within a 16-lane row (lane ^ 1,
          // lane ^ 2, then the mirror lane of the other half of 8), a
          // shuffle beyond it; every lane of the group ends with the word
          if constexpr (kLanesPerWord >= 2) w |= lane_dpp<0xB1>(w);   // quad_perm [1,0,3,2]
          if constexpr (kLanesPerWord >= 4) w |= lane_dpp<0x4E>(w);   // quad_perm [2,3,0,1]
          if constexpr (kLanesPerWord >= 8) w |= lane_dpp<0x141>(w);  // row_half_mirror
          if constexpr (kLanesPerWord >= 16) w |= lane_dpp<0x140>(w); // row_mirror
          if constexpr (kLanesPerWord >= 32) w |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(w), 16));
          if (s_out && lane % kLanesPerWord == 0) {
            const uint64_t off = static_cast<uint64_t>(t0 + k) * (ncl / 32) + i0 / 32;
            reinterpret_cast<uint32_t*>(a.spikes)[off] = w;
          }
        } else if (s_out) {
          const uint64_t off = static_cast<uint64_t>(t0 + k) * ncl + i0;
          store_pack<SRaw, VEC>(s_out + off, so);
        }
      }
    }
  }
  if (a.v_out) store_f32s<VEC>(a.v_out + i0, v);
  if (a.count_out) store_f32s<VEC>(a.count_out + i0, cnt);
}

template <typename Tag, int SPK, int VEC>
int launch(const LifArgs& a, bool has_res, hipStream_t stream) {
  const uint64_t threads = (static_cast<uint64_t>(a.NCL) + VEC - 1) / VEC;
  const uint64_t blocks = (threads + kBlock - 1) / kBlock;
  if (blocks == 0) return SNNK_OK;
  if (blocks > 0x7FFFFFFFull) return SNNK_EUNSUPPORTED;
  if (has_res)
    hipLaunchKernelGGL((lif_kernel<Tag, SPK, VEC, true>), dim3(blocks), dim3(kBlock), 0, stream, a);
  else
    hipLaunchKernelGGL((lif_kernel<Tag, SPK, VEC, false>), dim3(blocks), dim3(kBlock), 0, stream, a);
  return launch_status();
}

template <typename Tag, int SPK>
int dispatch_vec(const LifArgs& a, bool has_res, hipStream_t stream) {
  constexpr int VEC = 16 / sizeof(typename Tag::raw);
  // The vector path needs every per-step row to start on a 16-byte boundary
  // of the input and spike buffers.
  constexpr int SBYTES = SPK == 0 ? sizeof(typename Tag::raw) : (SPK == 1 ? 1 : 2);
  constexpr int SALIGN = SPK == 3 ? 4 : SBYTES * VEC;  // packed words: 4-byte stores
  bool vec_ok = (a.NCL % VEC == 0) && aligned(a.x, 16) &&
                (!has_res || aligned(a.residual, 16)) &&
                (a.spikes == nullptr || aligned(a.spikes, SALIGN)) &&
                aligned(a.v_init, 16) && aligned(a.v_out, 16) &&
                aligned(a.count_out, 16) &&
                (a.thr_mode != SNNK_THR_PER_NEURON || aligned(a.vth, 16));
  if (vec_ok) return launch<Tag, SPK, VEC>(a, has_res, stream);
  return launch<Tag, SPK, 1>(a, has_res, stream);
}

}  // namespace
}  // namespace snnk

using namespace snnk;

extern "C" int snnk_version(void) { return SNNK_VERSION; }

extern "C" const char* snnk_status_string(int status) {
  switch (status) {
    case SNNK_OK: return "ok";
    case SNNK_EINVAL: return "invalid argument";
    case SNNK_EUNSUPPORTED: return "unsupported configuration";
    case SNNK_EALIGN: return "misaligned pointer";
    case SNNK_EWORKSPACE: return "workspace missing or too small";
    case SNNK_ESCRATCH: return "needs more than the 32 MiB no-alloc scratch region (use the _ws entry point)";
    default: return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown status";
  }
}

extern "C" int snnk_lif_forward(const void* x, int32_t x_dtype,
                                const float* bias, const void* residual,
                                const float* vth, int32_t thr_mode, float vth_scalar,
                                const float* v_init, float* v_out,
                                void* spikes, int32_t spike_fmt, float* count_out,
                                int64_t T, int64_t NCL, int64_t C, int64_t HW,
                                int32_t channel_last,
                                float decay, float in_scale, float v_reset,
                                int32_t soft_reset, void* stream) {
  if (T < 0 || NCL < 0) return SNNK_EINVAL;
  if (T == 0 || NCL == 0) return SNNK_OK;
  if (x == nullptr) return SNNK_EINVAL;
  if (spikes == nullptr && count_out == nullptr && v_out == nullptr) return SNNK_EINVAL;
  if (thr_mode < SNNK_THR_SCALAR || thr_mode > SNNK_THR_PER_NEURON) return SNNK_EINVAL;
  if (thr_mode != SNNK_THR_SCALAR && vth == nullptr) return SNNK_EINVAL;
  if (spike_fmt < SNNK_SPIKE_SAME || spike_fmt > SNNK_SPIKE_BITS) return SNNK_EINVAL;
  if (spike_fmt == SNNK_SPIKE_BITS) {
    if (NCL % 32 != 0) return SNNK_EUNSUPPORTED;
    if (!aligned(spikes, 4)) return SNNK_EALIGN;
  }
  const bool need_c = bias != nullptr || thr_mode == SNNK_THR_PER_CHANNEL;
  if (need_c && (C <= 0 || HW <= 0)) return SNNK_EINVAL;
  if (C <= 0) C = 1;
  if (HW <= 0) HW = 1;

  LifArgs a{};
  a.x = x; a.bias = bias; a.residual = residual; a.vth = vth;
  a.v_init = v_init; a.v_out = v_out; a.spikes = spikes; a.count_out = count_out;
  a.T = T; a.NCL = NCL;
  a.C64 = static_cast<uint64_t>(C);
  a.HW64 = static_cast<uint64_t>(HW);
  a.use_div32 = (NCL <= 0xFFFFFFFFll) ? 1 : 0;
  a.C = static_cast<uint32_t>(C > 0xFFFFFFFFll ? 1 : C);
  a.div_c = make_fastdiv(a.C);
  a.div_hw = make_fastdiv(static_cast<uint32_t>(HW > 0xFFFFFFFFll ? 1 : HW));
  if (a.use_div32 && (C > 0xFFFFFFFFll || HW > 0xFFFFFFFFll)) a.use_div32 = 0;
  a.thr_mode = thr_mode; a.channel_last = channel_last ? 1 : 0;
  a.soft_reset = soft_reset ? 1 : 0;
  a.vth_scalar = vth_scalar; a.decay = decay; a.in_scale = in_scale; a.v_reset = v_reset;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool has_res = residual != nullptr;
  switch (x_dtype) {
    case SNNK_F32:
      return spike_fmt == SNNK_SPIKE_SAME ? dispatch_vec<F32, 0>(a, has_res, s)
             : spike_fmt == SNNK_SPIKE_U8 ? dispatch_vec<F32, 1>(a, has_res, s)
             : spike_fmt == SNNK_SPIKE_BF16 ? dispatch_vec<F32, 2>(a, has_res, s)
                                            : dispatch_vec<F32, 3>(a, has_res, s);
    case SNNK_BF16:
      return spike_fmt == SNNK_SPIKE_U8 ? dispatch_vec<BF16, 1>(a, has_res, s)
             : spike_fmt == SNNK_SPIKE_BITS ? dispatch_vec<BF16, 3>(a, has_res, s)
                                            : dispatch_vec<BF16, 0>(a, has_res, s);
    case SNNK_F16:
      return spike_fmt == SNNK_SPIKE_SAME ? dispatch_vec<F16, 0>(a, has_res, s)
             : spike_fmt == SNNK_SPIKE_U8 ? dispatch_vec<F16, 1>(a, has_res, s)
             : spike_fmt == SNNK_SPIKE_BF16 ? dispatch_vec<F16, 2>(a, has_res, s)
                                            : dispatch_vec<F16, 3>(a, has_res, s);
    default:
      return SNNK_EINVAL;
  }
}
