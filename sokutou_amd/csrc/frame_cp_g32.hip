// The code-predictor instantiations of the persistent kernel with i8g32 weights, the reference's int8 format (one
// fp16 scale per 32 weights of a row, qwen3/kernels.py:425-447; applied per 16-weight chunk inside the dots), for
// its serving default (qwen3/serve.py:55). sk_cp_frame checks the descriptor and calls here. A translation unit of
// its own, so the i8row code predictor's module keeps its generated code.
#include "frame_impl.h"

int sk_cp_frame_g32(const sk_cp_desc* d, hipStream_t st) {
  sk_talker_desc t;
  CpArgs cp;
  cp_launch_args(d, t, cp);
  if (d->keep_layers) return launch_frames<1024, 3072, 4, 2048, true, SK_WD_I8G32, true>(&t, cp, d->n_positions, st);
  return launch_frames<1024, 3072, 4, 2048, true, SK_WD_I8G32>(&t, cp, d->n_positions, st);
}
