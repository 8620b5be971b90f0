// The persistent frame kernel for the 0.6B talker (hidden 1024, intermediate 3072) with bf16 weights, the
// reference's Qwen3Kernels default (qwen3/kernels.py:487; no scales). Twice the bytes of int8: each stage's weights
// are loaded one exchange before their use (CfgW) instead of a layer ahead. A translation unit of its own, so the
// int8 kernels' modules keep their generated code.
#include "frame_impl.h"

int sk_talker_frames_bf16(const sk_talker_desc* d, int n_frames, hipStream_t st) {
  const CpArgs none{};
  return launch_frames<1024, 3072, 4, kTalkerV, false, SK_WD_BF16>(d, none, n_frames, st);
}
