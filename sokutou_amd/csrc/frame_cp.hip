// Entry point of the persistent kernel in code-predictor mode (sk_cp_frame, sk_cp_workspace_size); the kernel
// itself is in frame_impl.h. With desc->pair, launch_frames runs the paired pass of positions 0 and 1 as a launch
// of its own (k_frames with PAIRK) before the launch of the other positions. A translation unit of its own: the
// code predictor's instantiations do not share one with the talker's, so changes to either mode leave the other's
// generated code alone.
#include "frame_impl.h"

extern "C" int64_t sk_cp_workspace_size(int hidden, int inter, int pair) {
  if (hidden <= 0 || inter <= 0) return 0;
  (void)pair;  // the paired pass's and the projected input's cells are in the region whether used or not
  if (Layout(hidden, inter).total > kRegionCells) return 0;
  return Ws::kBytes;
}

extern "C" int sk_cp_frame(const sk_cp_desc* d, void* stream) {
  if (!d) return sk_set_error(SK_EINVAL, "sk_cp_frame: bad arguments");
  if (d->nq != kNQ || d->nkv != kNKV || d->vocab != 2048 || d->hidden != 1024 || d->inter != 3072 ||
      !(d->wd == SK_WD_I8ROW || d->wd == SK_WD_I8G32 || d->wd == SK_WD_BF16) || d->ct != SK_CT_BF16)
    return sk_set_error(SK_EUNSUPPORTED, "sk_cp_frame: needs hidden 1024, intermediate 3072, 16 q / 8 kv heads, "
                                         "vocab 2048, i8row, i8g32 or bf16 weights, bf16 cache");
  if (d->n_positions < 2 || d->n_positions > 64 || d->n_layers <= 0 || d->n_layers > Ws::kTraceLayers)
    return sk_set_error(SK_EUNSUPPORTED, "sk_cp_frame: 2..64 positions and 1..32 layers");
  if (!d->layers || !d->norm || !d->rope || !d->x0 || !d->id0 || !d->emb || !d->head_w || !d->head_s || !d->codes ||
      !d->workspace || d->emb0_rows <= 0)
    return sk_set_error(SK_EINVAL, "sk_cp_frame: null pointer");
  if (d->workspace_bytes < sk_cp_workspace_size(d->hidden, d->inter, d->pair))
    return sk_set_error(SK_EWORKSPACE, "sk_cp_frame: workspace too small");
  if (d->do_sample && (!d->seed || !d->counter || !(d->inv_temp > 0.f)))
    return sk_set_error(SK_EINVAL, "sk_cp_frame: sampling needs seed, counter and inv_temp > 0");
  if (d->proj_in != 0) {
    if (d->proj_in != 2048)
      return sk_set_error(SK_EUNSUPPORTED, "sk_cp_frame: a projected input must be 2048 wide (the 1.7B talker)");
    if (!d->proj_w || (!d->proj_s && d->wd != SK_WD_BF16))
      return sk_set_error(SK_EINVAL, "sk_cp_frame: projection weights or scales missing");
    if (d->pair) return sk_set_error(SK_EUNSUPPORTED, "sk_cp_frame: a projected code predictor runs unpaired");
    return sk_cp_frame_proj(d, (hipStream_t)stream);
  }
  if (d->wd == SK_WD_I8G32) return sk_cp_frame_g32(d, (hipStream_t)stream);
  if (d->wd == SK_WD_BF16) return sk_cp_frame_bf16(d, (hipStream_t)stream);
  sk_talker_desc t;
  CpArgs cp;
  cp_launch_args(d, t, cp);
  if (d->keep_layers) return launch_frames<1024, 3072, 4, 2048, true, SK_WD_I8ROW, true>(&t, cp, d->n_positions, (hipStream_t)stream);
  return launch_frames<1024, 3072, 4, 2048, true>(&t, cp, d->n_positions, (hipStream_t)stream);
}
