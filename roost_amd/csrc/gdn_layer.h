// Internal to the gfx950 Roost kernel library (not part of the C ABI): the CausalConv1d and GatedRmsNorm calls'
// admission and the convolution's state update, shared by those ops' own entry points (gdn_layer.hip) and the GDN
// decode-layer call that folds them into the recurrence (gated_delta_rule.hip).
#ifndef ROOST_AMD_GDN_LAYER_H_
#define ROOST_AMD_GDN_LAYER_H_

#include "contract.h"

namespace roost_layer {

// The rules of roost_causal_conv1d_run, reported under `op`.
RoostStatus AdmitConv(const RoostCausalConv1dParams& p, const char* op);

// The state update of an admitted CausalConv1d call alone: each sequence's slot keeps the last width - 1 inputs of
// [state, sequence]. Stream-ordered after everything that reads the old state.
RoostStatus ConvStateUpdate(const RoostCausalConv1dParams& p, hipStream_t s, const char* op);

// The rules of roost_gated_rms_norm_run, reported under `op`; *row_form (when not NULL) tells whether that run() serves
// the call with its single-pass kernel (one 16-byte vector per lane covers a row).
RoostStatus AdmitNorm(const RoostGatedRmsNormParams& p, const char* op, bool* row_form);

// The launches of an admitted GatedRmsNorm call, reported under `op`. stream_input: the single-pass kernel reads its
// input and gate rows with the non-temporal hint (the chunk layer, whose norm input the scan stored past the caches).
RoostStatus RunNorm(const RoostGatedRmsNormParams& p, hipStream_t s, bool stream_input, const char* op);

// RunNorm (input read as cached), then ConvStateUpdate, in one launch where both take their vector forms (a bf16
// single-pass norm over 128 columns; bf16 input with 2 to 4 taps and 16-byte aligned buffers), else as the two calls.
RoostStatus RunNormAndConvState(const RoostGatedRmsNormParams& np, const RoostCausalConv1dParams& cp, hipStream_t s,
                                const char* op);

}  // namespace roost_layer

#endif  // ROOST_AMD_GDN_LAYER_H_
