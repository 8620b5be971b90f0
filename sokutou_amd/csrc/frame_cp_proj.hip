// The code-predictor instantiations of the persistent kernel for a projected code predictor: the 1.7B Qwen3-TTS
// feeds its 1024-wide code predictor through small_to_mtp_projection from the talker's 2048-wide hidden state and
// embedding rows (qwen3/kernels.py:520-521, 629-637). Each position starts with a projection stage (CpProjIn): the
// input row staged in LDS, one projection row per compute wave (held in registers for the whole launch), the bias
// added, the projected vector exchanged as the stack's input. i8row, i8g32 and bf16 weights; sk_cp_frame checks the
// descriptor and calls here. A translation unit of its own, so the unprojected code predictor's modules keep their
// generated code.
#include "frame_impl.h"

namespace {
template <>
struct CpProjIn<1024, 3072> {
  static constexpr int value = 2048;
};
// as the unprojected bf16 code predictor (frame_cp_bf16.hip): the first half of each wave's gate/up rows goes out with
// o; the int8 instantiations do not spread their prefetch, so this applies to bf16 weights only
template <>
struct SplitGateUp<1024, 3072> {
  static constexpr bool value = true;
};
}  // namespace

int sk_cp_frame_proj(const sk_cp_desc* d, hipStream_t st) {
  sk_talker_desc t;
  CpArgs cp;
  cp_launch_args(d, t, cp);
  const int n = d->n_positions;
  if (d->wd == SK_WD_I8G32)
    return d->keep_layers ? launch_frames<1024, 3072, 4, 2048, true, SK_WD_I8G32, true>(&t, cp, n, st)
                          : launch_frames<1024, 3072, 4, 2048, true, SK_WD_I8G32>(&t, cp, n, st);
  if (d->wd == SK_WD_BF16)
    return d->keep_layers ? launch_frames<1024, 3072, 4, 2048, true, SK_WD_BF16, true>(&t, cp, n, st)
                          : launch_frames<1024, 3072, 4, 2048, true, SK_WD_BF16>(&t, cp, n, st);
  return d->keep_layers ? launch_frames<1024, 3072, 4, 2048, true, SK_WD_I8ROW, true>(&t, cp, n, st)
                        : launch_frames<1024, 3072, 4, 2048, true>(&t, cp, n, st);
}
