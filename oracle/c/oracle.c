/*
 * C restatement of the reference's CPU algorithms for the snnk parity tests.
 * TEST INFRASTRUCTURE ONLY: loaded by oracle/clib.py from tests/ and bench.py's
 * cpu_baseline leg; the product library never links it.
 *
 * Built with -ffp-contract=off so every product and sum is rounded to fp32
 * separately, as torch CPU evaluates the reference's expressions.
 */
#include <stdint.h>
#include <stddef.h>

/*
 * Multi-step IF/LIF over x[T][NCL] (fp32), restating
 * snn_compiler/kernels/neurons.py:491-502 (naive_if_lif) with the fused
 * bias / stateful extensions of snn_compiler/kernels/fused.py:101-114,424-441.
 *   bias: [C] or NULL, channel of flat i = (i/HW)%C
 *   vth:  [NCL] per-neuron thresholds or NULL (then vth_scalar)
 *   v_init: [NCL] or NULL; v_out: [NCL] or NULL; spikes: [T][NCL] 0/1 floats
 */
void oracle_lif_f32(const float* x, int64_t T, int64_t NCL,
                    const float* bias, int64_t C, int64_t HW,
                    const float* vth, float vth_scalar,
                    const float* v_init, float df, float sc,
                    int soft_reset, float v_reset,
                    float* spikes, float* v_out) {
  for (int64_t i = 0; i < NCL; ++i) {
    float v = v_init ? v_init[i] : 0.0f;
    const float th = vth ? vth[i] : vth_scalar;
    const float b = bias ? bias[(i / HW) % C] : 0.0f;
    for (int64_t t = 0; t < T; ++t) {
      float u = x[t * NCL + i];
      if (bias) u = u + b;
      float a = df * v;
      float c = sc * u;
      float h = a + c;
      int s = h >= th;
      spikes[t * NCL + i] = s ? 1.0f : 0.0f;
      if (soft_reset) v = s ? h - th : h;
      else v = s ? v_reset : h;
    }
    if (v_out) v_out[i] = v;
  }
}

/*
 * Pack {0,1} bytes src[rows][K] into dst[rows][ceil(K/32)] uint32 words:
 * bit k%32 of word k/32 holds element k (LSB first), tail bits zero.
 * Restates bitpack_N, snn_compiler/explore/attention/phase6b_bitpack.py:35-46.
 */
void oracle_pack_bits(const uint8_t* src, int64_t rows, int64_t K, uint32_t* dst) {
  const int64_t W = (K + 31) / 32;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t w = 0; w < W; ++w) {
      uint32_t word = 0;
      for (int j = 0; j < 32; ++j) {
        int64_t k = w * 32 + j;
        if (k < K && src[r * K + k]) word |= (uint32_t)1u << j;
      }
      dst[r * W + w] = word;
    }
  }
}

/*
 * Popcount GEMM over packed rows: C[m][n] = sum_w popcount(A[m][w] & B[n][w]).
 * Restates _ktv_popcount_kernel, snn_compiler/kernels/attention.py:217-233
 * (int32 counts; the reference stores them as fp32).  signed_w != 0 gives
 * 2*popc(A&B) - popc(A) (weights +1 where the bit is set, -1 elsewhere).
 * Rows [m0, m1) only, so a caller can check a bounded sample of rows.
 */
void oracle_popcount_gemm(const uint32_t* A, const uint32_t* B, int64_t m0, int64_t m1,
                          int64_t N, int64_t W, int signed_w, int32_t* Cout) {
#pragma omp parallel for schedule(static)
  for (int64_t m = m0; m < m1; ++m) {
    const uint32_t* a = A + m * W;
    int32_t rowpop = 0;
    for (int64_t w = 0; w < W; ++w) rowpop += __builtin_popcount(a[w]);
    for (int64_t n = 0; n < N; ++n) {
      const uint32_t* b = B + n * W;
      int32_t acc = 0;
      for (int64_t w = 0; w < W; ++w) acc += __builtin_popcount(a[w] & b[w]);
      Cout[(m - m0) * N + n] = signed_w ? 2 * acc - rowpop : acc;
    }
  }
}
