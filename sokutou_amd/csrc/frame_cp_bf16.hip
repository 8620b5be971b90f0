// The code-predictor instantiations of the persistent kernel with bf16 weights (layers and heads; the reference's
// Qwen3Kernels default, qwen3/kernels.py:487). sk_cp_frame checks the descriptor and calls here. A translation unit
// of its own, so the int8 code predictor's modules keep their generated code. The first half of each wave's
// gate/up rows goes out with o (SplitGateUp): 908 against 878 frames/s (the bf16 talker measured slower with it,
// 19.3 against 17.6 us per layer, and keeps the plain spread prefetch).
#include "frame_impl.h"

namespace {
template <>
struct SplitGateUp<1024, 3072> {
  static constexpr bool value = true;
};
}  // namespace

int sk_cp_frame_bf16(const sk_cp_desc* d, hipStream_t st) {
  sk_talker_desc t;
  CpArgs cp;
  cp_launch_args(d, t, cp);
  if (d->keep_layers) return launch_frames<1024, 3072, 4, 2048, true, SK_WD_BF16, true>(&t, cp, d->n_positions, st);
  return launch_frames<1024, 3072, 4, 2048, true, SK_WD_BF16>(&t, cp, d->n_positions, st);
}
