// Entry points of the persistent kernel in talker mode (sk_talker_workspace_size, sk_talker_frames) and the 0.6B
// talker's instantiations; the kernel itself is in frame_impl.h. The 1.7B talker runs the instantiations of
// frame17.hip (4 compute waves, register polls).
#include "frame_impl.h"

extern "C" int64_t sk_talker_workspace_size(int hidden, int inter) {
  if (hidden <= 0 || inter <= 0) return 0;
  // control words, trace stamps, then the 2 MB cell region at the first 2 MB boundary after them
  if (Layout(hidden, inter).talker_end > kRegionCells) return 0;
  return Ws::kBytes;
}

extern "C" int sk_talker_frames(const sk_talker_desc* d, int n_frames, void* stream) {
  if (!d || n_frames <= 0) return sk_set_error(SK_EINVAL, "sk_talker_frames: bad arguments");
  if (d->nq != kNQ || d->nkv != kNKV || d->vocab != kTalkerV || d->ct != SK_CT_BF16 ||
      !(d->wd == SK_WD_I8ROW || d->wd == SK_WD_I8G32 || d->wd == SK_WD_BF16))
    return sk_set_error(SK_EUNSUPPORTED, "sk_talker_frames: needs 16 q / 8 kv heads, vocab 3072, bf16 cache and i8row, "
                                         "i8g32 or bf16 weights");
  if (!d->layers || !d->norm || !d->head_w || (!d->head_s && d->wd != SK_WD_BF16) || !d->emb || !d->rope || !d->id0 ||
      !d->pos || !d->workspace)
    return sk_set_error(SK_EINVAL, "sk_talker_frames: null pointer");
  if (d->n_layers <= 0 || d->n_layers > Ws::kTraceLayers)
    return sk_set_error(SK_EUNSUPPORTED, "sk_talker_frames: 1..32 layers");
  if (d->workspace_bytes < sk_talker_workspace_size(d->hidden, d->inter))
    return sk_set_error(SK_EWORKSPACE, "sk_talker_frames: workspace too small");
  if (d->in_groups < 0 || d->in_groups > 64 ||
      (d->in_groups > 0 && (!d->in_tabs || !d->in_codes || !d->in_pad || d->in_rows <= 0 || n_frames != 1)))
    return sk_set_error(SK_EINVAL, "sk_talker_frames: talker_in input needs its tables, codes, pad, rows and one frame");
  if (d->do_sample && (!d->seed || !d->counter || !(d->inv_temp > 0.f)))
    return sk_set_error(SK_EINVAL, "sk_talker_frames: sampling needs seed, counter and inv_temp > 0");
  hipStream_t st = (hipStream_t)stream;
  const CpArgs none{};
  if (d->hidden == 1024 && d->inter == 3072) {
    if (d->wd == SK_WD_BF16) return sk_talker_frames_bf16(d, n_frames, st);
    return d->wd == SK_WD_I8G32 ? sk_talker_frames_g32(d, n_frames, st)
                                : launch_frames<1024, 3072, 4, kTalkerV, false>(d, none, n_frames, st);
  }
  if (d->hidden == 2048 && d->inter == 6144) return sk_talker_frames_2048(d, n_frames, st);
  return sk_set_error(SK_EUNSUPPORTED, "sk_talker_frames: shapes other than the 0.6B / 1.7B talker");
}
