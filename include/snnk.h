/*
 * snnk.h -- C ABI of libsnnk, the MI355X (gfx950) spiking-neural-network
 * inference kernel library.
 *
 * Every entry point follows the same contract:
 *   - returns int: 0 = ok, negative = invalid argument / unsupported
 *     configuration (see SNNK_E*), positive = the hipError_t raised by the
 *     launch;
 *   - takes the HIP stream (hipStream_t, passed as void*) and only enqueues
 *     work on it: no synchronisation, no host<->device copies;
 *   - never allocates: every buffer is owned by the caller and passed as a
 *     raw device pointer;
 *   - sizes are int64_t; tensors are dense row-major in the layout stated;
 *   - is re-entrant and thread-safe (no mutable global state), except
 *     snnk_conv3x3_bn_lif_noalloc, whose calls share one fixed scratch
 *     region per GPU (see there).
 *
 * The reference operator each entry point replaces is cited as
 * path:line inside Xarlley/Triton-Pass-Analysis.
 */
#ifndef SNNK_H_
#define SNNK_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define SNNK_OK            0
#define SNNK_EINVAL       -1   /* bad pointer / size / enum value          */
#define SNNK_EUNSUPPORTED -2   /* valid request this build does not cover   */
#define SNNK_EALIGN       -3   /* pointer alignment the kernel requires      */
#define SNNK_EWORKSPACE   -4   /* workspace missing or smaller than needed   */
#define SNNK_ESCRATCH     -5   /* needs more than the fixed no-alloc scratch  */

/* ---- element types --------------------------------------------------- */
#define SNNK_F32   0
#define SNNK_BF16  1
#define SNNK_F16   2
#define SNNK_U8    3
#define SNNK_I32   4

/* ---- spike output formats ------------------------------------------- */
#define SNNK_SPIKE_SAME  0   /* 0/1 in the input's element type            */
#define SNNK_SPIKE_U8    1   /* 0/1 as uint8                                */
#define SNNK_SPIKE_BF16  2   /* 0/1 as bf16 (input for the MFMA layers)      */
#define SNNK_SPIKE_BITS  3   /* packed: bit k%32 of uint32 word k/32 of each step
                                (NCL % 32 == 0); the layout snnk_binary_gemm reads */

/* ---- threshold modes (snn_compiler/kernels/neurons.py:66-68) --------- */
#define SNNK_THR_SCALAR      0
#define SNNK_THR_PER_CHANNEL 1
#define SNNK_THR_PER_NEURON  2

/* Library version (major*10000 + minor*100 + patch). */
int snnk_version(void);

/* Human-readable text for a status code returned by any entry point. */
const char* snnk_status_string(int status);

/*
 * Multi-step IF/LIF neuron, optionally fused with a per-channel bias, a
 * residual input, an initial / final membrane state and a spike-count
 * (rate) output.
 *
 * Replaces:
 *   if_lif                      snn_compiler/kernels/neurons.py:311-376
 *   fused_bias_if_lif           snn_compiler/kernels/fused.py:117-226
 *   fused_bias_if_lif_rate      snn_compiler/kernels/fused.py:303-382
 *   fused_bias_if_lif_stateful  snn_compiler/kernels/fused.py:444-507
 *
 * x        [T, NCL] elements of x_dtype (F32/BF16/F16); NCL = B*C*H*W
 * bias     [C] float or NULL; channel of flat index i is (i/HW)%C, or i%C
 *          when channel_last != 0
 * residual [T, NCL] of x_dtype or NULL
 * vth      [C] (PER_CHANNEL) or [NCL] (PER_NEURON) float; unused if SCALAR
 * v_init   [NCL] float or NULL (state starts at 0)
 * v_out    [NCL] float or NULL: membrane state after the last step
 * spikes   [T, NCL] in spike_fmt, [T, NCL/32] uint32 words for SNNK_SPIKE_BITS,
 *          or NULL (only count_out wanted)
 * count_out[NCL] float or NULL: sum over T of the spikes
 *
 * Per element and step t (all arithmetic fp32, rounded after every
 * operation, no fused multiply-add):
 *     u = x_t (+ bias[c]) (+ residual_t)
 *     v = decay*v + in_scale*u
 *     s = v >= threshold
 *     hard reset: v = s ? v_reset : v;  soft reset: v = s ? v - threshold : v
 */
int snnk_lif_forward(const void* x, int32_t x_dtype,
                     const float* bias, const void* residual,
                     const float* vth, int32_t thr_mode, float vth_scalar,
                     const float* v_init, float* v_out,
                     void* spikes, int32_t spike_fmt, float* count_out,
                     int64_t T, int64_t NCL, int64_t C, int64_t HW,
                     int32_t channel_last,
                     float decay, float in_scale, float v_reset,
                     int32_t soft_reset, void* stream);

/*
 * Pack {0,1} elements into uint32 words along K: element k of a row becomes
 * bit k%32 of word k/32 (least-significant first); bits past K are zero.
 *
 * Replaces:
 *   _pack_N / _pack_N_kernel  snn_compiler/kernels/attention.py:195-214,236-242
 *   bitpack_N (torch packer)  snn_compiler/explore/attention/phase6b_bitpack.py:35-46
 *
 * src  element (b, r, k) at src + b*stride_b + r*stride_r + k*stride_k
 *      (strides in elements; src_dtype F32/BF16/F16/U8; nonzero -> 1)
 * dst  [batch, rows, ceil(K/32)] uint32, dense
 */
int snnk_pack_bits(const void* src, int32_t src_dtype, uint32_t* dst,
                   int64_t batch, int64_t rows, int64_t K,
                   int64_t stride_b, int64_t stride_r, int64_t stride_k,
                   void* stream);

/* binary GEMM algorithms */
#define SNNK_BGEMM_AUTO    0   /* MFMA_F4 when M, N, K >= 128, else POPC       */
#define SNNK_BGEMM_POPC    1   /* VALU and + popcount-accumulate               */
#define SNNK_BGEMM_MFMA_I8 2   /* bits expanded to int8, v_mfma_i32_32x32x32_i8 */
#define SNNK_BGEMM_MFMA_F4 3   /* bits expanded to e2m1 0/1.0, MX fp4 MFMA      */

/*
 * Batched binary GEMM over bit-packed operands:
 *   C[b][m][n] = sum_k A[b][m][k] * B[b][n][k]              (signed_w == 0)
 *   C[b][m][n] = 2*sum_k A*B - sum_k A[b][m][k]              (signed_w != 0:
 *                B bit 1 means weight +1, bit 0 means -1)
 *
 * Replaces (generalised): spike_ktv_popcount / _ktv_popcount_kernel
 *   snn_compiler/kernels/attention.py:217-233,245-258
 *
 * A  [batch][M][lda] uint32 words (lda >= ceil(K/32)), B [batch][N][ldb],
 * C  [batch][M][ldc] of c_dtype (I32, or F32 as the reference returns);
 * strides between batch entries in words / elements (ignored if batch == 1).
 * Bits past K in the last word are ignored.
 */
int snnk_binary_gemm(const uint32_t* A, const uint32_t* B, void* C, int32_t c_dtype,
                     int64_t batch, int64_t M, int64_t N, int64_t K,
                     int64_t lda, int64_t ldb, int64_t ldc,
                     int64_t stride_a, int64_t stride_b, int64_t stride_c,
                     int32_t signed_w, int32_t algo, void* stream);

/*
 * Fused conv3x3 (stride 1, pad 1) + folded-BN bias + multi-step LIF
 * (+ 2x2 max-pool, stride 2), bf16 MFMA with fp32 accumulation; only spikes
 * are written.
 *
 * Replaces the layer pair
 *   FusedConvBNNeuron._conv_bn / forward   snn_compiler/nn/modules.py:324-357
 *     (F.conv2d + fused_bias_if_lif, snn_compiler/kernels/fused.py:101-114)
 *   followed by nn.MaxPool2d(2, 2)         snn_compiler/zoo/vgg.py:56,101-105
 *
 * x        [T][B][H][W][Cin] bf16 (NHWC per step), Cin % 32 == 0
 * w        [Cout][9*Cin] bf16, k = (kh*3 + kw)*Cin + cin, BN folded
 *          (fold_conv_bn, snn_compiler/kernels/fused.py:585-599); Cout % 32 == 0
 * bias     [Cout] fp32 or NULL
 * spikes_out [T][B][Ho][Wo][Cout] bf16 0/1, Ho = H/2, Wo = W/2 when pool
 * preact_out NULL, or [T][B][H][W][Cout] fp32 conv + bias instead of spikes
 *          (no LIF, pool must be 0): for numerical checks
 * LIF: v = decay*v + in_scale*(conv + bias); spike v >= v_threshold;
 *      hard reset to v_reset or soft reset (v -= v_threshold); state starts at 0.
 * tile_hint: -1 picks the tile shape from the problem size; 0..43 force one
 *          (29..38 keep the block's weights resident in LDS and take packed
 *          spike input only, Cin % 64 == 0; 39 and 40, 64x64 tiles with K over
 *          4 and 8 wave groups, and 43, 128x64 with 4 groups, take packed
 *          input only: SNNK_EUNSUPPORTED otherwise).
 */
int snnk_conv3x3_bn_lif(const uint16_t* x, const uint16_t* w, const float* bias,
                        uint16_t* spikes_out, float* preact_out,
                        int64_t T, int64_t B, int64_t H, int64_t W,
                        int64_t Cin, int64_t Cout, int32_t pool,
                        float decay, float in_scale, float v_threshold,
                        float v_reset, int32_t soft_reset, int32_t tile_hint,
                        void* stream);

/*
 * Linear + bias + multi-step LIF on bf16 MFMA (fp32 accumulation), the same
 * kernel as snnk_conv3x3_bn_lif run as a 1x1 conv over rows.
 *
 * Replaces FusedLinearNeuron.forward    snn_compiler/nn/modules.py:241-255
 *   (F.linear + fused_bias_if_lif) and linear_neuron, snn_compiler/kernels/fused.py:554-579;
 *   also the Conv1d-1x1 + BN + LIF projections of FusedSpikeAttention
 *   (snn_compiler/nn/attention.py:117-131).
 *
 * x [T][R][K] bf16 (R rows per step, e.g. batch or batch*tokens; R % 4 == 0,
 * K % 32 == 0), w [N][K] bf16 (nn.Linear layout, N % 32 == 0), bias [N] fp32
 * or NULL; spikes_out [T][R][N] bf16 0/1, or preact_out [T][R][N] fp32
 * (x.w^T + bias, no neuron).
 */
int snnk_linear_bias_lif(const uint16_t* x, const uint16_t* w, const float* bias,
                         uint16_t* spikes_out, float* preact_out, int64_t T,
                         int64_t R, int64_t K, int64_t N, float decay,
                         float in_scale, float v_threshold, float v_reset,
                         int32_t soft_reset, int32_t tile_hint, void* stream);

/*
 * Workspace variants of snnk_conv3x3_bn_lif and snnk_linear_bias_lif (same
 * arguments and results; no reference counterpart: the reference path
 * replaced is the same cuDNN conv / GEMM + fused LIF, fused.py:101-114).
 * They may split K across `splits` workgroups per output tile (0 = chosen
 * from the problem size, 1 = never): partial sums go to the caller's
 * workspace and the last workgroup of each tile sums them in split order
 * (deterministic) and runs the LIF epilogue.  The workspace starts with a
 * fixed 256 KB region of per-tile ticket counters that must be zero before
 * the first call (e.g. a zero-filled allocation); every call leaves it zero
 * again, so one workspace serves any sequence of calls, of any shapes, on
 * one stream -- calls that run concurrently must not share it.  16-byte x/w and 256-byte workspace
 * alignment.  *_ws_size returns the bytes needed for the same shape and
 * hints (0 when no split is chosen) or a negative status; a call with a
 * smaller workspace returns SNNK_EWORKSPACE.
 */
int snnk_conv3x3_bn_lif_ws(const uint16_t* x, const uint16_t* w, const float* bias,
                           uint16_t* spikes_out, float* preact_out,
                           int64_t T, int64_t B, int64_t H, int64_t W,
                           int64_t Cin, int64_t Cout, int32_t pool,
                           float decay, float in_scale, float v_threshold,
                           float v_reset, int32_t soft_reset, int32_t tile_hint,
                           int32_t splits, void* workspace, int64_t workspace_bytes,
                           void* stream);
int64_t snnk_conv3x3_bn_lif_ws_size(int64_t T, int64_t B, int64_t H, int64_t W,
                                    int64_t Cin, int64_t Cout, int32_t pool, int32_t preact,
                                    int32_t tile_hint, int32_t splits);
/*
 * snnk_conv3x3_bn_lif_ws without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 *
 * Same arguments, tiling and results as snnk_conv3x3_bn_lif_ws; the split-K
 * tickets and partial sums go to a fixed 32 MiB region of device memory inside
 * the library (one per GPU, held until the process ends).  The call allocates
 * nothing.  A plan that needs more than the region holds returns
 * SNNK_ESCRATCH (splits = 1 needs none).  Every call on one GPU shares that
 * GPU's region: calls that overlap on one GPU (two streams, two threads)
 * race.  The first call on a GPU also enqueues a fill kernel that zeroes the
 * region's ticket counters; every call leaves them at zero.
 */
int snnk_conv3x3_bn_lif_noalloc(const uint16_t* x, const uint16_t* w, const float* bias,
                                uint16_t* spikes_out, float* preact_out,
                                int64_t T, int64_t B, int64_t H, int64_t W,
                                int64_t Cin, int64_t Cout, int32_t pool,
                                float decay, float in_scale, float v_threshold,
                                float v_reset, int32_t soft_reset, int32_t tile_hint,
                                int32_t splits, void* stream);
int snnk_linear_bias_lif_ws(const uint16_t* x, const uint16_t* w, const float* bias,
                            uint16_t* spikes_out, float* preact_out, int64_t T,
                            int64_t R, int64_t K, int64_t N, float decay,
                            float in_scale, float v_threshold, float v_reset,
                            int32_t soft_reset, int32_t tile_hint, int32_t splits,
                            void* workspace, int64_t workspace_bytes, void* stream);
int64_t snnk_linear_bias_lif_ws_size(int64_t T, int64_t R, int64_t K, int64_t N,
                                     int32_t preact, int32_t tile_hint, int32_t splits);

/* ---- activation formats of the _act entry points ---------------------- */
#define SNNK_ACT_BF16 0   /* 0/1 as bf16, NHWC / [T][R][K]                       */
#define SNNK_ACT_BITS 1   /* packed: bit c%32 of uint32 word c/32 of each pixel's
                             (row's) channels, LSB first: [T][B][H][W][C/32]    */

/*
 * snnk_conv3x3_bn_lif_ws / snnk_linear_bias_lif_ws with a choice of
 * activation formats: x (x_fmt) and the spikes (out_fmt) as bf16 0/1 or as
 * packed bits (SNNK_ACT_BITS, 16x fewer bytes; the layout SNNK_SPIKE_BITS of
 * snnk_lif_forward gives for channels-last maps).  Packed x is expanded to
 * bf16 0/1 on its way into the MFMA operand stage; packed spikes are written
 * one 32-channel word per pixel and step.  Same results and workspace
 * contract as the _ws entry points; packed x has its own tile and split
 * plan (size the workspace with the *_act_ws_size functions below); LIF
 * only.  col_pool != 0 (Linear): the OR of each group of four adjacent output
 * columns, as snnk_linear_bias_lif_pool4_ws, with bf16 spikes out.  Packed
 * words need 4-byte alignment, bf16 x 16 bytes.
 *
 * Replaces the same layer pairs as snnk_conv3x3_bn_lif / snnk_linear_bias_lif,
 * with the bit-packed activation format of _pack_N
 * (snn_compiler/kernels/attention.py:195-214) between layers, the
 * "fused-LIF-pack" the reference lists as future work
 * (Document/Skill/snn-compiler-spiking-attention.md:232).
 */
int snnk_conv3x3_bn_lif_act(const void* x, int32_t x_fmt, const uint16_t* w, const float* bias,
                            void* spikes_out, int32_t out_fmt,
                            int64_t T, int64_t B, int64_t H, int64_t W,
                            int64_t Cin, int64_t Cout, int32_t pool,
                            float decay, float in_scale, float v_threshold,
                            float v_reset, int32_t soft_reset, int32_t tile_hint,
                            int32_t splits, void* workspace, int64_t workspace_bytes,
                            void* stream);
int snnk_linear_bias_lif_act(const void* x, int32_t x_fmt, const uint16_t* w, const float* bias,
                             void* spikes_out, int32_t out_fmt, int64_t T, int64_t R,
                             int64_t K, int64_t N, int32_t col_pool, float decay,
                             float in_scale, float v_threshold, float v_reset,
                             int32_t soft_reset, int32_t tile_hint, int32_t splits,
                             void* workspace, int64_t workspace_bytes, void* stream);
/* Pre-activation Linear on packed or bf16 spike rows: out [T][R][N] fp32 =
 * x W^T + bias (no neuron), x as in snnk_linear_bias_lif_act (x_fmt).  Size
 * the workspace with snnk_linear_bias_lif_act_ws_size (col_pool 0).
 * Replaces the output projection of the SSA block
 * (snn_compiler/nn/attention.py:160-164: proj_linear on the attention
 * spikes) when those spikes arrive packed. */
int snnk_linear_preact_act(const void* x, int32_t x_fmt, const uint16_t* w, const float* bias,
                           float* out, int64_t T, int64_t R, int64_t K, int64_t N,
                           int32_t tile_hint, int32_t splits, void* workspace,
                           int64_t workspace_bytes, void* stream);

/* Workspace bytes of the _act calls (packed x has its own tile / split plan,
 * so its workspace may differ from the bf16 one); col_pool as in
 * snnk_linear_bias_lif_pool4_ws (bf16 spikes out). */
int64_t snnk_conv3x3_bn_lif_act_ws_size(int64_t T, int64_t B, int64_t H, int64_t W,
                                        int64_t Cin, int64_t Cout, int32_t pool, int32_t x_fmt,
                                        int32_t tile_hint, int32_t splits);
int64_t snnk_linear_bias_lif_act_ws_size(int64_t T, int64_t R, int64_t K, int64_t N,
                                         int32_t x_fmt, int32_t col_pool, int32_t tile_hint,
                                         int32_t splits);

/*
 * snnk_linear_bias_lif_ws followed by an OR over each group of four adjacent
 * output columns: spikes_out [T][R][N/4] bf16, column c = max of the spikes of
 * columns 4c..4c+3 (the LIF runs per column first).  Same operands,
 * tiling and workspace contract (size it with snnk_linear_bias_lif_ws_size,
 * preact = 0).
 *
 * Replaces, for a 2x2 feature map, conv3x3 + BN + LIF + 2x2 max-pool
 *   (snn_compiler/nn/modules.py:324-357, snn_compiler/zoo/vgg.py:101-105):
 *   with every output pixel seeing all four input pixels, the conv is one
 *   dense matrix over (pixel, channel) -- w [(cout, pixel_out)][(pixel_in,
 *   cin)] -- and the pool is the OR over the four pixel columns of a channel.
 */
int snnk_linear_bias_lif_pool4_ws(const uint16_t* x, const uint16_t* w, const float* bias,
                                  uint16_t* spikes_out, int64_t T, int64_t R, int64_t K,
                                  int64_t N, float decay, float in_scale, float v_threshold,
                                  float v_reset, int32_t soft_reset, int32_t tile_hint,
                                  int32_t splits, void* workspace, int64_t workspace_bytes,
                                  void* stream);

/*
 * Classifier head averaged over time: out[r][n] = (1/T) * sum_t
 * (x[t][r] . w[n] + bias[n]), fp32 out [R][N]; same operands, tiling and
 * workspace contract as snnk_linear_bias_lif_ws (size it with
 * snnk_linear_bias_lif_ws_size(..., preact = 1, ...)).  Each step's sum is
 * accumulated in fp32 in step order and divided by T once.
 *
 * Replaces the last nn.Linear of the VGG classifier applied per step
 *   (snn_compiler/zoo/vgg.py:107-114) followed by the caller's mean over T
 *   (examples/vgg16_snn/benchmark_inference.py:68, `infer_model(xseq).mean(0)`).
 */
int snnk_linear_mean_t(const uint16_t* x, const uint16_t* w, const float* bias, float* out,
                       int64_t T, int64_t R, int64_t K, int64_t N, int32_t tile_hint,
                       int32_t splits, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The same head on packed spike words x [T][R][K/32] (bit k%32 of word k/32,
 * K % 32 == 0) for few outputs (N <= 64, SNNK_EUNSUPPORTED otherwise):
 * out[r][n] = (sum_k c[r][k] * w[n][k]) / T + bias[n], with c[r][k] the
 * spike count of input k over the T steps (the spikes are 0/1, so the T dot
 * products of the time average are one).  w [N][K] bf16, 16-byte aligned;
 * fp32 sums, reduced in a fixed order.  No workspace.
 *
 * Replaces, like snnk_linear_mean_t, the VGG classifier's last nn.Linear and
 *   the mean over T (snn_compiler/zoo/vgg.py:107-114,
 *   examples/vgg16_snn/benchmark_inference.py:68) when the layer before it
 *   writes packed spikes.
 */
int snnk_linear_mean_t_bits(const uint32_t* x, const uint16_t* w, const float* bias, float* out,
                            int64_t T, int64_t R, int64_t K, int64_t N, void* stream);

/*
 * Spike self-attention core: per (batch, head) and step t, integer
 * S = Q K^T and O = S V on int8 MFMA over {0,1} spikes (no softmax), then
 * a multi-step LIF on in_scale * O (in_scale = scale / tau for a LIF with
 * decay_input).  Counts are exact integers; with power-of-two scales the
 * membrane arithmetic is exact in fp32.
 *
 * Replaces the attention part of FusedSpikeAttention.forward
 *   snn_compiler/nn/attention.py:141-152: kv = K^T V (bmm or
 *   spike_ktv_popcount, snn_compiler/kernels/attention.py:245-258), then
 *   spike_av_lif (snn_compiler/kernels/attention.py:107-137); over integers
 *   (Q K^T) V == Q (K^T V).
 *
 * q, k, v: bf16 spikes; element (t, token row r = b*N + n, head h, dim dd) at
 *   ptr + t*step + r*row + h*d + dd (q/k/v may be column slices of one
 *   [T][B*N][3*H*d] projection output).  d % 8 == 0, d <= 128; pointers
 *   16-byte aligned, row and step strides multiples of 8, row strides below
 *   2^23 elements (SNNK_EUNSUPPORTED otherwise).  Up to 64 tokens and 64
 *   dims the counts are formed in the order (Q K^T) V on int8 MFMA; beyond,
 *   in the order Q (K^T V) on bf16 MFMA (equal over the integers; d*N < 2^24),
 *   where S is not formed: s_counts must then be NULL.
 * spikes_out: bf16, element (t, r, h*d + dd) at out + t*out_step + r*out_row + h*d + dd.
 * s_counts: NULL or int32 [T][B][H][N][N] (Q K^T); o_counts: NULL or int32
 *   [T][B][H][N][d] ((Q K^T) V).
 */
int snnk_spike_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         int64_t q_row, int64_t k_row, int64_t v_row,
                         int64_t q_step, int64_t k_step, int64_t v_step,
                         uint16_t* spikes_out, int64_t out_row, int64_t out_step,
                         int32_t* s_counts, int32_t* o_counts,
                         int64_t T, int64_t B, int64_t H, int64_t N, int64_t d,
                         float decay, float in_scale, float v_threshold,
                         float v_reset, int32_t soft_reset, void* stream);

/*
 * Fused (q @ kv) * scale -> multi-step LIF, the reference's linear attention
 * order: per batch*head and step t, a = q_t kv_t, v = decay*v + in_scale*a,
 * spike v >= v_threshold, hard reset to v_reset or soft reset.  The membrane
 * stays in registers across T; a is never written.
 *
 * Replaces spike_av_lif / _spike_av_lif_kernel
 *   snn_compiler/kernels/attention.py:49-137.
 *
 * q   [T][BH][N][d] of q_dtype (F32 / BF16 / F16), spikes 0/1
 * kv  [T][BH][d][d] of kv_dtype (F32 or I32), e.g. K^T V counts
 * spikes_out [T][BH][N][d] of q_dtype
 * d <= 128.  q @ kv runs on bf16 MFMA with fp32 accumulation and kv as three
 * bf16 parts whose sum is exactly its fp32 value: every product is exact, so
 * integer kv (sums below 2^24) gives the exact count; real kv gives an fp32
 * sum.  q values other than 0/1 are rounded to bf16.
 */
/*
 * snnk_spike_attention on packed spikes: q, k, v and the output are uint32
 * words of LSB-first bits (the _pack_N convention).  Head h of q, k and v
 * starts at bit h*in_head_bits of a token row (in_head_bits >= d, a multiple
 * of 8: in_head_bits = d reads the rows a packed projection writes); head h
 * of the output starts at word h*out_head_words (>= ceil(d/32)), its bits
 * past d written as zero.  Row and step strides count words; 4-byte
 * alignment.  N <= 64 and d <= 64 (the quadratic core).  The same counts and
 * spikes as snnk_spike_attention.  Replaces the same reference code as
 * snnk_spike_attention (snn_compiler/nn/attention.py:133-164), on the packed
 * format of _pack_N (snn_compiler/kernels/attention.py:195-214).
 */
int snnk_spike_attention_packed(const uint32_t* q, const uint32_t* k, const uint32_t* v,
                                int64_t q_row, int64_t k_row, int64_t v_row,
                                int64_t q_step, int64_t k_step, int64_t v_step,
                                int64_t in_head_bits, uint32_t* spikes_out,
                                int64_t out_row, int64_t out_step, int64_t out_head_words,
                                int32_t* s_counts, int32_t* o_counts,
                                int64_t T, int64_t B, int64_t H, int64_t N, int64_t d,
                                float decay, float in_scale, float v_threshold,
                                float v_reset, int32_t soft_reset, void* stream);

int snnk_spike_av_lif(const void* q, int32_t q_dtype, const void* kv, int32_t kv_dtype,
                      void* spikes_out, int64_t T, int64_t BH, int64_t N, int64_t d,
                      float decay, float in_scale, float v_threshold, float v_reset,
                      int32_t soft_reset, void* stream);

/*
 * Input layer: a static image presented at all T steps.  conv3x3 (pad 1)
 * in fp32 computed once per pixel, then T LIF steps on that constant input.
 * Replaces the first FusedConvBNNeuron of VGGSNN (snn_compiler/zoo/vgg.py:57-68)
 * fed with the image repeated over T.
 *
 * image [B][Cin][H][W] fp32 (NCHW); w [Cout][Cin][3][3] fp32 (BN folded);
 * bias [Cout] fp32 or NULL; spikes_out [T][B][H][W][Cout] bf16 0/1.
 */
int snnk_conv3x3_image_lif(const float* image, const float* w, const float* bias,
                           uint16_t* spikes_out, int64_t T, int64_t B, int64_t Cin,
                           int64_t H, int64_t W, int64_t Cout, float decay,
                           float in_scale, float v_threshold, float v_reset,
                           int32_t soft_reset, void* stream);

/*
 * snnk_conv3x3_image_lif with a choice of spike format: SNNK_ACT_BF16 as
 * above, or SNNK_ACT_BITS, packed words [T][B][H][W][Cout/32] (bit c%32 of
 * word c/32; Cout % 32 == 0, 4-byte alignment), the input format of
 * snnk_conv3x3_bn_lif_act.
 */
int snnk_conv3x3_image_lif_act(const float* image, const float* w, const float* bias,
                               void* spikes_out, int32_t out_fmt, int64_t T, int64_t B,
                               int64_t Cin, int64_t H, int64_t W, int64_t Cout, float decay,
                               float in_scale, float v_threshold, float v_reset,
                               int32_t soft_reset, void* stream);

/*
 * Layout change [N][C][HW] -> [N][HW][C] with conversion to bf16
 * (src_dtype F32 / BF16 / F16 / U8; fp32 rounds to nearest even).
 */
int snnk_to_nhwc_bf16(const void* src, int32_t src_dtype, uint16_t* dst,
                      int64_t N, int64_t C, int64_t HW, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* SNNK_H_ */
