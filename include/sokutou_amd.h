/* sokutou_amd: C-ABI of the MI355X (gfx950) Qwen3-TTS talker decode step.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed as `void*` (torch's
 * `torch.cuda.current_stream().cuda_stream`), enqueues its kernels on that stream and returns immediately:
 * no host synchronisation, no host reads of device memory and no allocation, so every call can be captured in
 * a HIP graph. The caller owns every buffer. Return value: SK_OK (0) or a negative SK_E* code; the message of
 * the last failure on the calling thread is `sk_last_error()`.
 *
 * Each function names the reference kernel it replaces (paths relative to the Soyomi66/sokutou repository).
 * In the reference those are `extern "C" __global__` CUDA kernels launched through CuPy with a grid, a block
 * and a tuple of raw pointers (`Qwen3Kernels._launch`, qwen3/kernels.py:575-577); here the launch shape is
 * chosen inside the library and the call takes only the kernel's own arguments.
 */
#ifndef SOKUTOU_AMD_H
#define SOKUTOU_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------------------------------------- */
#define SK_OK 0
#define SK_EINVAL (-1)       /* bad shape, format or null pointer (the reference's asserts)                */
#define SK_ELAUNCH (-2)      /* the HIP launch failed                                                       */
#define SK_EUNSUPPORTED (-3) /* a feature this build does not provide                                       */
#define SK_EWORKSPACE (-4)   /* workspace too small                                                          */
#define SK_EDEVICE (-5)      /* not a gfx950 device                                                          */

/* ---- weight formats (`wd` of _Lin, qwen3/kernels.py:434-444, plus per-channel int8) -------------------- */
#define SK_WD_I8ROW 0 /* int8 [N,K] + bf16 scale per output row                                          */
#define SK_WD_I8G32 1 /* int8 [N,K] + fp16 scale per 32 consecutive K elements ([N, K/32])               */
#define SK_WD_BF16 2  /* bf16 [N,K]                                                                       */
#define SK_WD_F32 3   /* fp32 [N,K]                                                                       */

/* ---- cache / embedding element types (the reference's ct_t: bf16, or f32 under ACT_F32) --------------- */
#define SK_CT_BF16 0
#define SK_CT_F32 1

#define SK_MAX_K 8192 /* largest GEMV input length (1.7B down projection is 6144)                         */
#define SK_MAX_V 4096 /* largest sampler vocabulary (qwen3/sampler.py:162)                               */

/* Library and device checks. sk_device_check returns SK_OK when the current HIP device is gfx950 (the
 * reference's sm_80 gate, qwen3/kernels.py:492-493). */
const char* sk_version(void);
const char* sk_last_error(void);
int sk_device_check(void);

/* out = W · (h ⊙ nw) · rsqrt(mean(h²) + eps). With swiglu != 0 the rows of W are interleaved gate/up and
 * out[n] = silu(row 2n) · row 2n+1 (N/2 outputs). K % 512 == 0, K <= SK_MAX_K.
 * policy 1 streams the weights with nontemporal loads (read once per frame), 0 uses ordinary loads.
 * Replaces rms_gemv(h, nw, eps, W, S, out, N, K, swiglu, split, policy) (qwen3/kernels.py:271-275). */
int sk_rms_gemv(const float* h, const float* nw, float eps, const void* W, const uint16_t* S, float* out, int N, int K,
                int swiglu, int wd, int policy, void* stream);

/* out = W · x (+ bias) (+ out when accumulate != 0). bias may be NULL.
 * Replaces gemv(x, W, S, bias, out, N, K, accumulate, split, policy) (qwen3/kernels.py:301-305). */
int sk_gemv(const float* x, const void* W, const uint16_t* S, const float* bias, float* out, int N, int K,
            int accumulate, int wd, int policy, void* stream);

/* out = h · rsqrt(mean(h²) + eps) · nw over K elements.
 * Replaces rmsnorm(h, nw, eps, out, K) (qwen3/kernels.py:313-319). */
int sk_rmsnorm(const float* h, const float* nw, float eps, float* out, int K, void* stream);

/* out[i] = float(table[idx[0] * dim + i]); idx is a device int64.
 * Replaces embed(table, idx, out, dim) (qwen3/kernels.py:322-326). */
int sk_embed(const void* table, const int64_t* idx, float* out, int dim, int ct, void* stream);

/* out[i] = Σ_g tabs[g][codes[g] * dim + i] + pad[i]; tabs is a device array of G table addresses.
 * Replaces talker_in(tabs, codes, pad, out, dim, G) (qwen3/kernels.py:329-336). */
int sk_talker_in(const uint64_t* tabs, const int64_t* codes, const void* pad, float* out, int dim, int G, int ct,
                 void* stream);

/* Bytes of scratch that sk_attn needs for nkv kv heads and caches of max_len positions: the error word (bytes 0..3),
 * per-head arrival counters, then split-K partials. The error word and the counters must be zero before the first
 * call; sk_attn leaves the counters zero. One workspace sized for the longest cache serves calls with any shorter
 * max_len. */
int64_t sk_attn_workspace_size(int nq, int nkv, int max_len);

/* One-token GQA decode attention. qkv is [nq·128 | nkv·128 | nkv·128] fp32; for each kv head: per-head RMSNorm
 * of k (weight kn) and q (weight qn), rotate-half RoPE from rope[pos] = [cos 64 | sin 64], K and V stored at
 * position pos of Kc/Vc ([nkv][max_len][128], element type ct), q scaled by 1/sqrt(128), softmax over positions
 * 0..pos, out = [nq·128] fp32. pos = (pos_ptr ? *pos_ptr : 0) + pos_add, read on the device. nq == 2·nkv.
 * The cache length is split across blocks and merged with a log-sum-exp (online softmax) combine. A position
 * outside [0, max_len) sets the workspace's error word to 5 (it stays set until the caller clears it) and the call
 * reads and writes nothing else.
 * Replaces attn(qkv, qn, kn, eps, rope, Kc, Vc, pos_ptr, pos_add, max_len, nq, nkv, out)
 * (qwen3/kernels.py:341-414). */
int sk_attn(const float* qkv, const float* qn, const float* kn, float eps, const float* rope, void* Kc, void* Vc,
            const int64_t* pos_ptr, int pos_add, int max_len, int nq, int nkv, float* out, void* workspace,
            int64_t workspace_bytes, int ct, void* stream);

/* sk_attn without a workspace, for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. Same arguments and results as
 * sk_attn, except that the split-K scratch (arrival counters and partials) lives in a static device array of the
 * library, 260 KiB per device, held until the process ends: at most 16 kv heads (more is SK_EINVAL). err (nullable,
 * device int32) receives 5 when the position lies outside [0, max_len) (the call then writes nothing else) and is
 * left alone otherwise. The call allocates nothing; its first call on a device looks up the array and launches a
 * small kernel that clears the counters, so make that first call outside graph capture (later calls may be
 * captured: the merging block leaves the counters at zero for the next call or replay). Every call on one device
 * shares the array: calls that overlap on one device (concurrent streams or threads) race and must be serialised by
 * the caller. */
int sk_attn_noalloc(const float* qkv, const float* qn, const float* kn, float eps, const float* rope, void* Kc, void* Vc,
                    const int64_t* pos_ptr, int pos_add, int max_len, int nq, int nkv, float* out, int* err, int ct,
                    void* stream);

/* One sampling step over V <= SK_MAX_V fp32 logits, writing the chosen id to out[0] (int64).
 * talker != 0 applies the talker processor first (repetition penalty on seen, suppressed ids, EOS blocked while
 * ngen < min_new) and then updates the device state: id0 = id, seen[id] = 1, ngen += 1, pos += 1.
 * do_sample == 0 is greedy argmax with the lowest index winning ties. seen / suppress are bool (1 byte) arrays,
 * NULL when unused; seed / counter are device uint64 (used only when sampling).
 * Replaces sample(logits, V, inv_temp, top_k, do_sample, seen, rep_pen, suppress, ngen, min_new, eos, seed,
 * counter, out, talker, id0, pos) (qwen3/sampler.py:37-159). do_sample != 0 scales by inv_temp (> 0), keeps the
 * entries at or above the top_k-th largest (top_k <= 0 or >= V keeps all) that are not -inf and picks the largest
 * v - log(-log(u)), u from Philox4x32-10 with counter (index, *counter) and key *seed; *counter += 1 after the draw
 * (seed / counter are device uint64). The same seed and counter give the reference kernel's pick. */
int sk_sample(const float* logits, int V, float inv_temp, int top_k, int do_sample, uint8_t* seen, float rep_pen,
              const uint8_t* suppress, int64_t* ngen, int min_new, int eos, const uint64_t* seed, uint64_t* counter,
              int64_t* out, int talker, int64_t* id0, int64_t* pos, void* stream);

/* ---- whole frames in one launch ------------------------------------------------------------------------- */

/* One decoder layer's device pointers (i8row weights: int8 [N,K] + bf16 scale per row). kc/vc are this
 * layer's caches [nkv][max_len][128] bf16. */
typedef struct sk_layer_desc {
  const void* qkv_w;        /* [(nq + 2 nkv) * 128, H], q rows then k rows then v rows */
  const uint16_t* qkv_s;
  const void* o_w;          /* [H, nq * 128] */
  const uint16_t* o_s;
  const void* gu_w;         /* [2 I, H], row 2n gate n, row 2n + 1 up n */
  const uint16_t* gu_s;
  const void* down_w;       /* [H, I] */
  const uint16_t* down_s;
  const float* in_norm;     /* [H] */
  const float* post_norm;   /* [H] */
  const float* qn;          /* [128] */
  const float* kn;          /* [128] */
  void* kc;
  void* vc;
} sk_layer_desc;

/* A talker and its frame state, all device pointers. `layers` is a device array of n_layers descriptors.
 * id0 / pos / next_id0 / ngen / seen are the reference's frame state (qwen3/fast.py:99-106); out (optional)
 * receives the id chosen in each frame; logits (optional) the raw logits of the last frame; layer_out (optional,
 * [n_layers][H]) the residual after every layer of the last frame. */
typedef struct sk_talker_desc {
  int n_layers, hidden, inter, nq, nkv, vocab, max_len, wd, ct;
  float eps;
  const sk_layer_desc* layers;
  const float* norm;        /* final RMSNorm weight [H] */
  const void* head_w;       /* codec head [vocab, H] */
  const uint16_t* head_s;
  const void* emb;          /* input embedding table [vocab, H] bf16 */
  const float* rope;        /* [max_len][cos 64 | sin 64] */
  int64_t* id0;
  int64_t* pos;
  int64_t* next_id0;
  int64_t* out;
  uint8_t* seen;
  int64_t* ngen;
  const uint8_t* suppress;
  float rep_pen;
  int min_new;
  int eos;
  int talker_processor;     /* 1: repetition penalty / suppression / EOS block before the argmax */
  float* logits;
  float* layer_out;
  void* workspace;
  int64_t workspace_bytes;
  /* Optional talker_in input (qwen3/kernels.py:328-336, 686-687), for a talker fed by a code predictor: when
   * in_groups > 0 the frame's input is Σ_g in_tabs[g][in_codes[g]] + in_pad instead of the embedding row of id0
   * (in_tabs: device array of in_groups bf16 tables [rows, hidden]; in_codes: device int64 [in_groups], code 0
   * < vocab and the others < in_rows; in_pad: bf16 [hidden]). Needs n_frames == 1 (the next frame's codes come
   * from the code predictor). final_out (optional, fp32 [hidden]) receives the frame's final residual after
   * the final norm (the rmsnorm output the code predictor's position 0 takes). Zero / NULL when unused. */
  const uint64_t* in_tabs;
  const int64_t* in_codes;
  const void* in_pad;
  int in_groups;
  int in_rows;
  float* final_out;
  /* Sampled picks (the draw of sk_sample with do_sample != 0): when do_sample != 0 each frame's pick is the
   * Gumbel-max over the processed logits times inv_temp (> 0) that are at or above the top_k-th largest
   * (top_k <= 0 keeps all), with Philox4x32-10 keyed by *seed and draw *counter + frame; *counter advances by
   * the number of draws (device uint64). */
  int do_sample;
  float inv_temp;
  int top_k;
  const uint64_t* seed;
  uint64_t* counter;
} sk_talker_desc;

/* Bytes of workspace sk_talker_frames needs. It must be zero before the first call and must be zeroed again
 * after a call that reported an error (its first 4 bytes hold the error code, 0 when healthy). */
int64_t sk_talker_workspace_size(int hidden, int inter);

/* Places the exchange cells of a zeroed sk_talker_frames / sk_cp_frame workspace: measures which 4 KB page of each
 * 32 KB period of the workspace's cell region is nearest each XCD (every XCD reads its own copy of the cells, on its
 * nearest page) and records the result in the workspace, where every later launch reads it. One launch of 256
 * one-wave workgroups, about 0.3 ms, stream-ordered; call it after each zeroing of the workspace, outside graph
 * capture, with no frame launch on the same workspace in flight. Without it (or when the measurement is not
 * consistent across the region) the launches use a fixed placement: the same results, slower exchanges. No
 * counterpart in the reference, whose kernels exchange nothing between launches (its per-op launches,
 * qwen3/kernels.py:619-627, pass activations through global memory at kernel boundaries). */
int sk_frames_place(void* workspace, int64_t workspace_bytes, void* stream);

/* n_frames greedy talker frames in ONE launch: for each frame, embedding row of id0 -> n_layers decoder layers
 * -> final RMSNorm -> codec head -> (processor) -> argmax -> next id, with the frame state advanced on the
 * device exactly as the fused sampler advances it (id0, next_id0, seen, ngen, pos += 1 per frame).
 * 256 persistent workgroups (one per CU, grouped by XCD: kv head x on XCD x) exchange activations through the
 * workspace. Supports the 0.6B (H 1024, I 3072) and 1.7B (H 2048, I 6144) talkers: 16 q / 8 kv heads, vocab
 * 3072, i8row, i8g32 or bf16 weights (head_s may be null for bf16), bf16 cache, max_len <= 2048, a
 * 256-CU device.
 * Replaces, for greedy decoding, the talker half of Qwen3Kernels._frame (qwen3/kernels.py:676-685): talker_in /
 * embed, _layers (rms_gemv, attn, gemv, rms_gemv, gemv per layer, qwen3/kernels.py:619-627), rmsnorm, gemv
 * (codec_head) and sample (qwen3/sampler.py:37-159 with do_sample = 0). */
int sk_talker_frames(const sk_talker_desc* desc, int n_frames, void* stream);

/* The code predictor of one frame, all device pointers. `layers` holds its decoder stack (kc / vc are
 * [nkv][n_positions][128] bf16). emb / head_w / head_s are device arrays of n_positions pointers: position 0 takes
 * the vector x0 (the talker's last hidden state after its final norm) and has no head; position g >= 1 takes row
 * codes[g - 1] of table emb[g] (bf16 [rows][hidden]; codes[0] = *id0 must be < emb0_rows) and ends in the final
 * norm, head g (int8 [vocab][hidden] + bf16 row scales) and a greedy pick (lowest index wins ties) into codes[g]. */
typedef struct sk_cp_desc {
  int n_layers, hidden, inter, nq, nkv, vocab, n_positions, wd, ct;
  float eps;
  const sk_layer_desc* layers;
  const float* norm;          /* final RMSNorm weight [hidden], applied before every head */
  const float* rope;          /* [n_positions][cos 64 | sin 64] */
  const float* x0;            /* position 0 input, fp32 [hidden] */
  const int64_t* id0;         /* code 0 */
  int emb0_rows;
  const void* const* emb;
  const void* const* head_w;
  const void* const* head_s;
  int64_t* codes;             /* [n_positions]: codes[0] = code 0, codes[g] = the pick at position g */
  float* logits;              /* optional: head output of the last position (before the pick) */
  float* layer_out;           /* optional: [n_layers][hidden] residual after every layer at the last position */
  void* workspace;            /* sk_talker_workspace_size(hidden, inter) bytes, zeroed as for sk_talker_frames */
  int64_t workspace_bytes;
  /* Sampled sub-codes (no processor): as sk_talker_desc; position g >= 1 draws with counter *counter + g - 1,
   * and *counter advances by n_positions - 1. */
  int do_sample;
  float inv_temp;
  int top_k;
  const uint64_t* seed;
  uint64_t* counter;
  /* Nonzero: the layer weights are loaded through the caches (they are read once per position, 16 times per frame,
   * and stay in L2 / the Infinity Cache); 0: streamed with non-temporal loads, as the heads always are. The
   * reference's l2_keep_mb policy (qwen3/kernels.py:525-542), for the code predictor's layers as a whole. */
  int keep_layers;
  /* Nonzero: positions 0 and 1 run as one pass with two rows per stage, in a launch of their own before the
   * other positions' (each layer's weights read once for both; the reference's cp_pair, qwen3/kernels.py:600-617);
   * the workspace is then sk_cp_workspace_size(hidden, inter, 1) bytes. 0: one position after the other, one
   * launch. Either gives the same codes up to fp32 summation order. */
  int pair;
  /* Optional input projection, the code predictor's small_to_mtp_projection (qwen3/kernels.py:520-521, 629-637):
   * with proj_in > 0 the position inputs are proj_in wide (x0 fp32 [proj_in], the emb tables bf16 [rows][proj_in])
   * and each position's input to the stack is proj_w . input + proj_b, a gemv over proj_w ([hidden][proj_in] in the
   * weight format wd, proj_s its scales as for the layers, null for bf16) with the fp32 bias proj_b ([hidden],
   * nullable). proj_in 0: the inputs are hidden wide and enter the stack as they are. Supported: proj_in 2048 (the
   * 1.7B talker's width) with pair = 0. */
  int proj_in;
  const void* proj_w;
  const uint16_t* proj_s;
  const float* proj_b;
} sk_cp_desc;

/* Bytes of workspace sk_cp_frame needs: sk_talker_workspace_size(hidden, inter), whose cell region also holds the
 * cells of a projected input and, for pair = 1, the second row's. sk_frames_place serves it too. */
int64_t sk_cp_workspace_size(int hidden, int inter, int pair);

/* All positions of the code predictor of one frame in ONE launch, or two with desc->pair (the paired pass of
 * positions 0 and 1, then the rest), of the persistent kernel of sk_talker_frames in its code-predictor mode:
 * greedy sub-codes 1..n_positions-1. Supports the Qwen3-TTS code predictor shape:
 * hidden 1024, intermediate 3072, 16 q / 8 kv heads, vocab 2048, i8row, i8g32 or bf16 weights (layers and heads;
 * head_s entries may be 0 for bf16), bf16 cache, a 256-CU device.
 * Replaces, for greedy sub-codes, the code-predictor loop of Qwen3Kernels._frame (qwen3/kernels.py:666-675) with
 * _cp_first / _cp_input (qwen3/kernels.py:629-655), _layers (619-627), rms_gemv over cp_heads[g - 1] and sample
 * (qwen3/sampler.py:37-159 with do_sample = 0, no processor). Positions 0 and 1 run one after the other, or as one
 * paired pass (desc->pair: _cp_first with cp_pair, qwen3/kernels.py:641-646, and _cp_layers_pair, 600-617, whose
 * rms_gemv2 / gemv2 read each weight once for both rows, qwen3/kernels.py:276-310). */
int sk_cp_frame(const sk_cp_desc* desc, void* stream);


/* ---- batched decode: up to 16 streams per step on the matrix cores -------------------------------------------
 * The reference decodes one stream (qwen3/fast.py:146); these entry points have no reference kernel to replace.
 * They run the same layer math as sk_talker_frames over a batch, with every projection an M = 16 skinny GEMM on
 * bf16 MFMA: int8 weights (exact in bf16) in the tile layout of sk_tile_weights, activations passed as
 * sk_batch_terms() bf16 planes whose sum is the fp32 value. */

/* Number of bf16 terms per activation value (planes of every batched GEMM input). */
int sk_batch_terms(void);

/* Rewrites int8 weights [N, K] (row-major) into the batched GEMM's tile layout (same size): tile (g, c) is
 * 1 KiB at byte (g * K/64 + c) * 1024 and holds W[16 g + n][64 c + 16 j + e] at byte 16 (n + 16 j) + e.
 * N % 16 == 0, K % 64 == 0. */
int sk_tile_weights(const void* w, void* tiled, int N, int K, void* stream);

/* Workspace bytes of sk_bgemm for an [N, K] projection (split-K partial sums and per-tile arrival counters; zero
 * it once, every call leaves the counters zero). */
int64_t sk_bgemm_workspace_size(int N, int K);

/* One M = 16 projection. x: bf16 planes [terms][16][K]; w_tiled / s: tiled int8 weights [N, K] + bf16 row scales.
 * ssp (optional, [np][16]): partial sums of squares of the residual whose normalised copy x is; when given, row m
 * is multiplied by rsqrt(Σ_q ssp[q][m] / K + eps) after the dot product (the fused RMSNorm of rms_gemv,
 * qwen3/kernels.py:180-186, 224). mode 0: out[16][N] = result (fp32). mode 1: rows interleaved gate/up,
 * act = planes [terms][16][N/2] of silu(gate) * up. mode 2: out[16][N] += result (the residual), then xn = planes
 * [terms][16][N] of out ⊙ nw and ssp_out[N/16][16] = per 16-column partial sums of squares of out.
 * K in {512, 1024, 2048, 3072, 4096, 6144}; N % 16 == 0 (N % 32 == 0 for mode 1). Row groups of 16 outputs go
 * to workgroups in sets of up to 4, and K is split over as many workgroups as it takes to occupy the GPU; the
 * split sums are added in a fixed order by the last workgroup of each set, so results are deterministic. */
int sk_bgemm(const void* x, const float* ssp, int np, float eps, const void* w_tiled, const uint16_t* s, int N, int K,
             int mode, float* out, void* act, void* xn, const float* nw, float* ssp_out, void* workspace,
             int64_t workspace_bytes, void* stream);

/* Workspace bytes of sk_batch_attn (zeroed once; its first 4 bytes are the error word, 5 = a position out of
 * range). */
int64_t sk_batch_attn_workspace_size(int nkv);

/* Decode attention of `batch` streams, each at its own position pos[b] (device int64) of its own caches
 * Kc / Vc [batch][nkv][max_len][128] bf16, with the math of sk_attn (per-head q/k RMSNorm, rotate-half RoPE,
 * bf16 K/V append at pos[b], softmax over positions 0..pos[b]). qkv: [16][(nq + 2 nkv) * 128] fp32; att: bf16
 * planes [terms][16][nq * 128] (the input of the o projection). Split over (stream, kv head, 64 positions) with a
 * log-sum-exp merge; max_len <= 4096.
 * Replaces, per stream, attn (qwen3/kernels.py:338-414). */
int sk_batch_attn(const float* qkv, const float* qn, const float* kn, float eps, const float* rope, void* Kc, void* Vc,
                  const int64_t* pos, int batch, int max_len, int nq, int nkv, void* att, void* workspace,
                  int64_t workspace_bytes, void* stream);

/* A batch of talker streams. layers is a HOST array of n_layers descriptors whose weights are tiled
 * (sk_tile_weights) and whose caches kc / vc are [batch][nkv][max_len][128] bf16; head_w is tiled too. ids / pos /
 * nstep are device int64 [batch]: each stream's current token, the position it is written at, and how many picks
 * it has made; codes is [max_frames][16] int64 (codes[f][b] = pick f of stream b). logits (optional) receives
 * [16][vocab] of the last step, layer_out (optional) [n_layers][16][hidden] residuals of the last step. */
typedef struct sk_batch_desc {
  int n_layers, hidden, inter, nq, nkv, vocab, batch, max_len;
  float eps;
  const sk_layer_desc* layers;
  const float* norm;
  const void* head_w;
  const uint16_t* head_s;
  const void* emb;            /* input embedding table [vocab, hidden] bf16 */
  const float* rope;          /* [max_len][cos 64 | sin 64] */
  int64_t* ids;
  int64_t* pos;
  int64_t* codes;
  int64_t* nstep;
  int max_frames;
  float* logits;
  float* layer_out;
  void* workspace;
  int64_t workspace_bytes;
} sk_batch_desc;

/* Workspace bytes for the batched step; zero it once before the first call (its first 4 bytes are the error
 * word: 0 healthy, 5 a position or token out of range, 6 more picks than max_frames). */
int64_t sk_batch_workspace_size(int hidden, int inter, int nq, int nkv, int vocab);

/* Loads each stream's input for the next step: h = emb[ids[b]] and its normalised planes. */
int sk_batch_embed(const sk_batch_desc* desc, void* stream);

/* One decode step for every stream: n_layers x (qkv GEMM, ragged split-K attention with KV append at pos[b] and
 * its merge, o GEMM, gate/up GEMM, down GEMM), final RMSNorm + head GEMM, greedy pick per stream (lowest index on
 * ties), then codes / ids / nstep / pos advance and the picked rows are embedded for the next step.
 * 6 n_layers + 2 launches. */
int sk_batch_frame(const sk_batch_desc* desc, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SOKUTOU_AMD_H */
