// Packed-spike input variants of the fused conv3x3 / Linear + LIF kernel
// (conv_kernel.h with PK = true), in a translation unit of their own so that
// they compile in parallel with conv.hip.  The A operand is read as packed
// words (bit c%32 of word c/32 of a pixel's channels, the layout the LIF and
// conv epilogues write with SNNK_ACT_BITS) and expanded to bf16 0/1 in LDS.
#include "conv_kernel.h"

namespace snnk {

int dispatch_packed(const ConvArgs& a, const Plan& p, void* workspace, hipStream_t s, bool pool,
                    int taps, bool preact) {
  if (preact) return dispatch<false, MODE_PREACT, 1, true>(a, p, workspace, s);  // fp32 x.W^T + b
  if (taps == 1) {  // with pool: the OR of each group of four adjacent columns
    return pool ? dispatch<true, MODE_LIF, 1, true>(a, p, workspace, s)
                : dispatch<false, MODE_LIF, 1, true>(a, p, workspace, s);
  }
  if (pool) return dispatch<true, MODE_LIF, 9, true>(a, p, workspace, s);
  return dispatch<false, MODE_LIF, 9, true>(a, p, workspace, s);
}

}  // namespace snnk
