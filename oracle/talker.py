"""CPU restatement (numpy, float32) of the Qwen3-TTS talker decode step: the oracle.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, never by the product package. Every function cites the reference code it restates
(paths are relative to the Soyomi66/sokutou repository).

Numerics follow the reference exactly where it fixes a rounding point:
  * the residual stream, the normalised GEMV input and all accumulation are float32
    (qwen3/kernels.py:10, 155-190, 552-566);
  * the KV cache and the embedding table are bf16, rounded to nearest even
    (``f2bf``, qwen3/kernels.py:42-57, 364-366);
  * the current token's K is stored as bf16 first and read back rounded for its own score
    (qwen3/kernels.py:364, 386-391);
  * the RMSNorm scale ``inv`` is applied after the dot product in the fused GEMV
    (qwen3/kernels.py:180-186, 224) and as ``h * inv * w`` in the standalone norm (qwen3/kernels.py:317-318).
Summation order inside a dot product is not fixed by the reference (it changes with the launch shape,
qwen3/gemv2_bench.py:157-172), so the oracle uses BLAS order.

How each function is pinned (independent checks, in ``tests/test_oracle.py``):
  * ``bf16_round``           - torch ``.to(torch.bfloat16)`` on every fp32 bit class, NaN rule by hand.
  * ``quantize_rowwise``     - crafted rows (exact .5 ties, zero rows, max clamp) + brute-force Python loop.
  * ``quantize_g32``         - crafted groups + brute force; fp16 scale rounding against numpy float16.
  * ``rope_table``           - closed form cos/sin in float64.
  * ``rms_gemv``/``gemv``    - float64 brute force on small shapes.
  * ``attention``            - transformers' Qwen3Attention (eager) with the same weights, f32 cache;
                               T=1 gives out = V; uniform K gives mean(V).
  * ``decoder_layer``        - transformers' Qwen3DecoderLayer (f32 cache) within 1e-5.
  * ``process_logits``/``argmax_first`` - crafted ties, NaN, all -inf; restated from qwen3/sampler.py:50-65, 129-149.
  * ``philox4x32_10``        - the Random123 known-answer vectors of philox4x32_10.
  * ``topk_threshold``       - brute force (count of strictly larger keys < k <= count of keys >= it).
  * ``gumbel_uniform``       - PARITY UNPINNED for the draw sequence: its Philox counter layout (index, draw lo,
                               draw hi, 0x51), key order and uniform mapping ((r0 >> 8) + 0.5) * 2^-24 are read
                               from qwen3/sampler.py:118-125. The reference holds no vectors of its draws, and its
                               CUDA kernel (compiled by CuPy NVRTC) cannot run here. The Philox function itself is
                               pinned by the known-answer vectors, and ``sample_draw``'s law by a chi-square test;
                               neither would catch a swapped counter word.
  * ``sample_draw``          - the empirical law of many draws against softmax over the top-k (chi-square), and
                               the keep rule by hand on crafted ties / -inf / NaN.
"""

from __future__ import annotations

import numpy as np

HD = 128
F32 = np.float32
INV_SQRT_HD = F32(0.08838834764831845)  # qwen3/kernels.py:378


# ---------------------------------------------------------------------------------------------------------
# storage rounding
# ---------------------------------------------------------------------------------------------------------
def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round to nearest even, NaN -> 0x7fc0 (qwen3/kernels.py:42-47)."""
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    r = r.astype(np.uint16)
    r[nan] = np.uint16(0x7FC0)
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit pattern -> fp32 by a 16-bit shift (``bf``, qwen3/kernels.py:41)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(F32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 value after a round trip through bf16 storage (``STC`` then ``LDC``, qwen3/kernels.py:54-56)."""
    return bf16_to_f32(bf16_bits(x))


# ---------------------------------------------------------------------------------------------------------
# weight quantisation
# ---------------------------------------------------------------------------------------------------------
def quantize_rowwise(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel int8 with a bf16 scale: ``s = bf16(max(max_k|w|/127, 1e-12))``,
    ``q = clamp(rne(w/s), -127, 127)``.

    The reference's per-row precedent is ``i8row`` in qwen3/gemv_bench.py:136-137 (fp32 row scale); the bf16
    scale and the clamp-then-round order follow its i8g32 quantiser (qwen3/kernels.py:438-442).
    Returns (q int8 [N,K], scale as bf16 bits uint16 [N]).
    """
    w = np.ascontiguousarray(w, dtype=F32)
    amax = np.abs(w).max(axis=1)
    s_bits = bf16_bits(np.maximum(amax / F32(127), F32(1e-12)))
    s = bf16_to_f32(s_bits)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint(w / s[:, None])
    q = np.nan_to_num(q, nan=0.0)
    q = np.clip(q, -127, 127).astype(np.int8)
    return q, s_bits


def quantize_g32(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """i8g32: int8 plus an fp16 scale per 32 consecutive K elements of a row (qwen3/kernels.py:438-442).

    ``sc = fp16(max(max|g|/127, 1e-12))``; ``q = clamp(round(g/sc), +-127)``. A group whose fp16 scale
    underflows to 0 (an all-zero group) divides 0/0; the reference leaves the int8 cast of NaN to the
    platform, here it is defined as 0. Returns (q int8 [N,K], scales as fp16 bits uint16 [N, K/32]).
    """
    w = np.ascontiguousarray(w, dtype=F32)
    N, K = w.shape
    g = w.reshape(N, K // 32, 32)
    sc = np.maximum(np.abs(g).max(axis=2) / F32(127), F32(1e-12)).astype(np.float16)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint(g / sc.astype(F32)[..., None])
    q = np.nan_to_num(q, nan=0.0, posinf=127.0, neginf=-127.0)
    q = np.clip(q, -127, 127).astype(np.int8).reshape(N, K)
    return q, sc.view(np.uint16)


def dequant_rowwise(q: np.ndarray, s_bits: np.ndarray) -> np.ndarray:
    """W = q * s, exact in fp32 (8-bit by 8-bit significands)."""
    return q.astype(F32) * bf16_to_f32(s_bits)[:, None]


def dequant_g32(q: np.ndarray, s_bits: np.ndarray) -> np.ndarray:
    """W = q * s_group, exact in fp32 (8-bit by 11-bit significands)."""
    N, K = q.shape
    s = s_bits.view(np.float16).astype(F32)
    return (q.astype(F32).reshape(N, K // 32, 32) * s[..., None]).reshape(N, K)


def quantize(w: np.ndarray, wd: str):
    """Dispatch on the weight format name used by ``_Lin`` (qwen3/kernels.py:434-444).
    Returns (stored weights, scales or None, dequantised fp32 weights)."""
    w = np.ascontiguousarray(w, dtype=F32)
    if wd == "i8row":
        q, s = quantize_rowwise(w)
        return q, s, dequant_rowwise(q, s)
    if wd == "i8g32":
        q, s = quantize_g32(w)
        return q, s, dequant_g32(q, s)
    if wd == "bf16":
        b = bf16_bits(w)
        return b, None, bf16_to_f32(b)
    if wd == "f32":
        return w, None, w.copy()
    raise ValueError(wd)


# ---------------------------------------------------------------------------------------------------------
# layer pieces
# ---------------------------------------------------------------------------------------------------------
def rope_table(inv_freq: np.ndarray, max_len: int) -> np.ndarray:
    """[pos][cos 64 | sin 64] with fp32 angle ``pos * inv_freq`` (qwen3/kernels.py:473-476).
    cos/sin are evaluated in float64 and rounded once to fp32."""
    inv = np.asarray(inv_freq, dtype=F32)
    f = np.arange(max_len, dtype=F32)[:, None] * inv[None, :]
    f64 = f.astype(np.float64)
    return np.concatenate([np.cos(f64), np.sin(f64)], axis=1).astype(F32)


def rmsnorm(h: np.ndarray, nw: np.ndarray, eps: float) -> np.ndarray:
    """``out = h * rsqrt(mean(h^2) + eps) * nw`` (qwen3/kernels.py:312-319)."""
    h = h.astype(F32)
    inv = F32(1.0) / np.sqrt(np.dot(h, h) / F32(h.size) + F32(eps), dtype=F32)
    return (h * inv) * nw.astype(F32)


def bf16_terms(x: np.ndarray, n: int) -> np.ndarray:
    """x as the sum of ``n`` bf16 values (``t_0 = bf16(x)``, ``t_i = bf16(x - t_0 - ... - t_{i-1})``, each
    difference exact in fp32), summed back in fp32: the input the batched path's matrix cores see. n = 0 is x."""
    x = np.asarray(x, dtype=F32)
    if n <= 0:
        return x
    r, acc = x.copy(), np.zeros_like(x)
    for _ in range(n):
        t = bf16_round(r)
        acc = acc + t
        r = r - t
    return acc


def _act(x: np.ndarray, act_bf16) -> np.ndarray:
    # act_bf16: False/0 exact fp32 inputs, True/1 one bf16 term, n: a sum of n bf16 terms
    return bf16_terms(x, int(act_bf16))


def rms_gemv(h: np.ndarray, nw: np.ndarray, eps: float, W: np.ndarray, swiglu: bool = False,
             act_bf16: bool = False) -> np.ndarray:
    """``y = W (h*nw) * rsqrt(mean(h^2)+eps)``; with swiglu the rows are interleaved gate/up and
    ``out[n] = g/(1+exp(-g)) * u`` from rows 2n, 2n+1 (qwen3/kernels.py:255-275, 267).
    ``act_bf16`` rounds the staged vector ``h*nw`` to bf16 before the product (the batched path's rounding point).
    ``h`` may also be a batch [B, K] (one row per stream)."""
    h = h.astype(F32)
    if h.ndim == 2:
        ss = np.einsum("bk,bk->b", h, h).astype(F32)
        inv = F32(1.0) / np.sqrt(ss / F32(h.shape[1]) + F32(eps), dtype=F32)
        y = (_act(h * nw.astype(F32)[None, :], act_bf16) @ W.T) * inv[:, None]
        if swiglu:
            g, u = y[:, 0::2], y[:, 1::2]
            return (g / (F32(1.0) + np.exp(-g))) * u
        return y
    inv = F32(1.0) / np.sqrt(np.dot(h, h) / F32(h.size) + F32(eps), dtype=F32)
    y = (W @ _act(h * nw.astype(F32), act_bf16)) * inv
    if swiglu:
        g, u = y[0::2], y[1::2]
        return (g / (F32(1.0) + np.exp(-g))) * u
    return y


def gemv(x: np.ndarray, W: np.ndarray, bias: np.ndarray | None = None, out: np.ndarray | None = None,
         act_bf16: bool = False) -> np.ndarray:
    """``out (+)= W x (+ bias)`` (qwen3/kernels.py:283-305): bias then the accumulated value are added to the
    dot product, in that order. ``act_bf16`` rounds x to bf16 first; ``x`` may be a batch [B, K]."""
    x = _act(x.astype(F32), act_bf16)
    v = x @ W.T if x.ndim == 2 else W @ x
    if bias is not None:
        v = v + bias.astype(F32)
    if out is not None:
        v = v + out
    return v


def _head_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    # per-head RMSNorm over hd=128: x * rsqrt(sum(x^2)/HD + eps) * w (qwen3/kernels.py:355-360, 371-375)
    ss = np.einsum("hd,hd->h", x, x).astype(F32)
    inv = F32(1.0) / np.sqrt(ss / F32(HD) + F32(eps), dtype=F32)
    return (x * inv[:, None]) * w[None, :]


def _rot(x: np.ndarray, c: np.ndarray, s: np.ndarray) -> np.ndarray:
    # rotate-half RoPE on index d & 63: d<64 -> x*c - x[d+64]*s, else x*c + x[d-64]*s (qwen3/kernels.py:363-364, 377-378)
    r = np.concatenate([-x[:, 64:], x[:, :64]], axis=1)
    cc = np.concatenate([c, c])
    ss = np.concatenate([s, s])
    return x * cc[None, :] + r * ss[None, :]


def attention(qkv: np.ndarray, qn: np.ndarray, kn: np.ndarray, eps: float, rope: np.ndarray,
              Kc: np.ndarray, Vc: np.ndarray, pos: int, nq: int, nkv: int, cache_bf16: bool = True) -> np.ndarray:
    """One-token GQA decode attention with fused q/k RMSNorm, RoPE and KV append (qwen3/kernels.py:338-414).

    ``Kc``/``Vc`` are fp32 arrays [nkv, max_len, 128] holding the cache values (bf16-representable when
    ``cache_bf16``); position ``pos`` is overwritten in place. q head ``h`` reads kv head ``h // (nq/nkv)``.
    Returns the attention output [nq*128] fp32.
    """
    assert nq % nkv == 0
    q = qkv[: nq * HD].reshape(nq, HD).astype(F32)
    k = qkv[nq * HD:(nq + nkv) * HD].reshape(nkv, HD).astype(F32)
    v = qkv[(nq + nkv) * HD:(nq + 2 * nkv) * HD].reshape(nkv, HD).astype(F32)
    c, s = rope[pos, :64], rope[pos, 64:]
    kr = _rot(_head_norm(k, kn.astype(F32), eps), c, s)
    rnd = bf16_round if cache_bf16 else (lambda a: a.astype(F32))
    Kc[:, pos, :] = rnd(kr)
    Vc[:, pos, :] = rnd(v)
    qr = _rot(_head_norm(q, qn.astype(F32), eps), c, s) * INV_SQRT_HD
    T = pos + 1
    rep = nq // nkv
    out = np.empty((nq, HD), dtype=F32)
    for h in range(nq):
        kv = h // rep
        sc = Kc[kv, :T, :] @ qr[h]
        m = sc.max()
        e = np.exp(sc - m)
        out[h] = (e @ Vc[kv, :T, :]) / e.sum(dtype=F32)
    return out.reshape(-1)


def decoder_layer(h: np.ndarray, L: dict, eps: float, rope: np.ndarray, Kc: np.ndarray, Vc: np.ndarray, pos: int,
                  nq: int, nkv: int, cache_bf16: bool = True, act_bf16: bool = False) -> np.ndarray:
    """One decoder layer on the fp32 residual ``h`` (qwen3/kernels.py:619-627):
    rms_gemv(qkv) -> attn -> gemv(o, +=h) -> rms_gemv(gu, swiglu) -> gemv(down, +=h).
    ``L`` holds dequantised fp32 matrices ``qkv`` [(nq+2nkv)*128, H], ``o``, ``gu`` (gate/up rows interleaved),
    ``down`` and the fp32 norm vectors ``in_norm``, ``post_norm``, ``qn``, ``kn``. ``act_bf16`` rounds every
    projection input to bf16 (the batched path)."""
    qkv = rms_gemv(h, L["in_norm"], eps, L["qkv"], act_bf16=act_bf16)
    att = attention(qkv, L["qn"], L["kn"], eps, rope, Kc, Vc, pos, nq, nkv, cache_bf16)
    h = gemv(att, L["o"], out=h, act_bf16=act_bf16)
    act = rms_gemv(h, L["post_norm"], eps, L["gu"], swiglu=True, act_bf16=act_bf16)
    return gemv(act, L["down"], out=h, act_bf16=act_bf16)


# ---------------------------------------------------------------------------------------------------------
# sampling (greedy)
# ---------------------------------------------------------------------------------------------------------
def process_logits(logits: np.ndarray, seen: np.ndarray | None, rep_pen: float, suppress: np.ndarray | None,
                   ngen: int, min_new: int, eos: int) -> np.ndarray:
    """Talker logits processor: repetition penalty on ``seen`` (``v<0 ? v*p : v/p``), suppressed ids -> -inf,
    EOS -> -inf while ``ngen < min_new`` (qwen3/sampler.py:50-61; qwen3/fast.py:154-166)."""
    v = logits.astype(F32).copy()
    p = F32(rep_pen)
    if seen is not None:
        pen = np.where(v < 0, v * p, v / p)
        v = np.where(seen.astype(bool), pen, v).astype(F32)
    if suppress is not None:
        v[suppress.astype(bool)] = -np.inf
    if ngen < min_new and 0 <= eos < v.size:
        v[eos] = -np.inf
    return v


def order_key(v: np.ndarray) -> np.ndarray:
    """fp32 -> uint32 key with the same order as the values (sign bit set for positives, all bits flipped for
    negatives) (``fkey``, qwen3/sampler.py:21-24)."""
    u = np.ascontiguousarray(v, dtype=F32).view(np.uint32)
    return np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)


PHILOX_M = (0xD2511F53, 0xCD9E8D57)
PHILOX_W = (0x9E3779B9, 0xBB67AE85)


def philox4x32_10(ctr: np.ndarray, key: np.ndarray) -> np.ndarray:
    """Philox4x32 with 10 rounds (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
    SC'11): per round two 32x32->64-bit products of the counter words 0 and 2 with the published multipliers, the
    high halves xored with the other words and the key, then the key bumped by the Weyl constants.
    ``ctr`` [..., 4] and ``key`` [..., 2] uint32 (broadcast); returns [..., 4] uint32. The reference's sampler
    uses this generator (qwen3/sampler.py:25-34)."""
    c = [np.asarray(ctr[..., i], dtype=np.uint64) for i in range(4)]
    k0 = np.asarray(key[..., 0], dtype=np.uint64)
    k1 = np.asarray(key[..., 1], dtype=np.uint64)
    m32 = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        p0 = np.uint64(PHILOX_M[0]) * c[0]
        p1 = np.uint64(PHILOX_M[1]) * c[2]
        c = [((p1 >> np.uint64(32)) ^ c[1] ^ k0) & m32, p1 & m32, ((p0 >> np.uint64(32)) ^ c[3] ^ k1) & m32, p0 & m32]
        k0 = (k0 + np.uint64(PHILOX_W[0])) & m32
        k1 = (k1 + np.uint64(PHILOX_W[1])) & m32
    return np.stack(np.broadcast_arrays(*c), axis=-1).astype(np.uint32)


def topk_threshold(v: np.ndarray, top_k: int) -> int:
    """Order key of the top_k-th largest value (0 keeps everything when top_k <= 0 or top_k >= V). The reference
    finds it by a 4-pass 8-bit radix select over the keys (qwen3/sampler.py:67-112); the result is the key of
    the k-th largest entry, ties included, which this computes by sorting."""
    if top_k <= 0 or top_k >= v.size:
        return 0
    return int(np.sort(order_key(v))[::-1][top_k - 1])


def gumbel_uniform(V: int, seed: int, counter: int) -> np.ndarray:
    """The uniform in (0, 1) of every index for one draw: ``(r0 >> 8) + 0.5`` scaled by 2^-24 (exact in fp32), with
    r = Philox4x32-10(counter = (i, draw lo, draw hi, 0x51), key = (seed lo, seed hi)) (qwen3/sampler.py:118-123)."""
    i = np.arange(V, dtype=np.uint32)
    ctr = np.stack([i, np.full(V, counter & 0xFFFFFFFF, np.uint32), np.full(V, (counter >> 32) & 0xFFFFFFFF, np.uint32),
                    np.full(V, 0x51, np.uint32)], axis=1)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], dtype=np.uint32)
    r = philox4x32_10(ctr, key)
    return ((r[:, 0] >> np.uint32(8)).astype(F32) + F32(0.5)) * F32(1.0 / 16777216.0)


def sample_draw(v: np.ndarray, inv_temp: float, top_k: int, seed: int, counter: int, exact: bool = False):
    """One sampled pick from processed logits ``v`` (qwen3/sampler.py:47-154 with do_sample = 1): v * inv_temp,
    keep the entries whose key is at least the top_k threshold and that are not -inf, then the argmax of
    v - log(-log(u)) (Gumbel-max: the same law as softmax sampling over the kept entries), lowest index on ties,
    index 0 if nothing is kept. Returns (index, perturbed values) with the perturbation in fp32, or in float64
    when ``exact`` (to measure how close the top two are)."""
    x = np.asarray(v, dtype=F32) * F32(inv_temp)
    thr = topk_threshold(x, top_k)
    keep = (order_key(x) >= np.uint32(thr)) & (x != -np.inf)
    u = gumbel_uniform(x.size, seed, counter)
    if exact:
        g = x.astype(np.float64) - np.log(-np.log(u.astype(np.float64)))
    else:
        g = x - np.log(-np.log(u)).astype(F32)
    g = np.where(keep, g, -np.inf)
    ok = ~np.isnan(g) & keep
    if not ok.any():
        return 0, g
    m = g[ok].max()
    return int(np.flatnonzero(ok & (g == m))[0]), g


def argmax_first(v: np.ndarray) -> int:
    """Greedy pick: the largest value, lowest index on ties; NaN never wins; all -inf picks index 0
    (qwen3/sampler.py:114-149)."""
    v = np.asarray(v, dtype=F32)
    ok = ~np.isnan(v)
    if not ok.any():
        return 0
    m = v[ok].max()
    return int(np.flatnonzero(ok & (v == m))[0])


# ---------------------------------------------------------------------------------------------------------
# whole model
# ---------------------------------------------------------------------------------------------------------
class TalkerOracle:
    """Talker decode over dequantised fp32 weights (the synthetic greedy loop: embedding row -> 28 layers ->
    final RMSNorm -> codec head -> argmax -> next embedding row).

    Frame composition follows the talker half of ``Qwen3Kernels._frame`` (qwen3/kernels.py:676-685) with the
    ``embed`` kernel (qwen3/kernels.py:321-326) as the input, which is how ``_cp_first`` feeds id0
    (qwen3/kernels.py:642). ``weights`` is a dict with ``layers`` (list of dicts as in ``decoder_layer``),
    ``norm`` [H], ``head`` [V, H] fp32 (dequantised), ``emb`` [V, H] (bf16 values as fp32), ``rope``,
    ``eps``, ``nq``, ``nkv``; ``K``/``V`` are fp32 caches [layers, nkv, max_len, 128].
    """

    def __init__(self, weights: dict, K: np.ndarray, V: np.ndarray, cache_bf16: bool = True):
        self.w = weights
        self.K = K
        self.V = V
        self.cache_bf16 = cache_bf16

    def forward(self, h: np.ndarray, pos: int, layer_out: list | None = None) -> np.ndarray:
        w = self.w
        h = h.astype(F32)
        for i, L in enumerate(w["layers"]):
            h = decoder_layer(h, L, w["eps"], w["rope"], self.K[i], self.V[i], pos, w["nq"], w["nkv"], self.cache_bf16)
            if layer_out is not None:
                layer_out.append(h.copy())
        return h

    def logits(self, h: np.ndarray) -> np.ndarray:
        return gemv(rmsnorm(h, self.w["norm"], self.w["eps"]), self.w["head"])

    def step(self, token: int, pos: int, layer_out: list | None = None) -> tuple[int, np.ndarray]:
        x = self.w["emb"][token].astype(F32)
        lg = self.logits(self.forward(x, pos, layer_out))
        return argmax_first(lg), lg

    def greedy(self, token: int, pos: int, frames: int, record: bool = False):
        codes, logits = [], []
        for f in range(frames):
            token, lg = self.step(token, pos + f)
            codes.append(token)
            if record:
                logits.append(lg)
        return codes, logits


class CodePredictorOracle:
    """One frame of the code predictor over dequantised fp32 weights (the greedy sub-code loop of
    ``Qwen3Kernels._frame``, qwen3/kernels.py:666-675, with ``_cp_first`` 641-655 and ``_cp_input`` 629-639):

      * position 0 takes the talker's last hidden state ``x0`` (``_cp_input(ph32)``), position 1 the talker
        embedding row of code 0 (``embed(temb, id0)``), position g >= 2 row ``codes[g-1]`` of code table g - 2
        (``cemb[g-2]``); each input goes through ``_cp_input`` (qwen3/kernels.py:629-637): the projection
        ``small_to_mtp_projection`` as a gemv with its bias when the weights hold ``proj`` ([H, talker width])
        and ``proj_b``, else the identity (both stacks equally wide);
      * each position runs the decoder stack at position g over a cache that starts empty for the frame;
      * position g >= 1 ends in ``rms_gemv(h, norm, eps, heads[g-1])`` and a greedy pick (lowest index on ties;
        the sub-codes get no processor, qwen3/kernels.py:671-674).

    Positions 0 and 1 may be computed as one pair in the reference (``_cp_layers_pair``, 600-617); the result is
    the same row by row, so they are computed one after the other here. ``weights``: ``layers`` (as in
    ``decoder_layer``), ``norm``, ``heads`` (list of [V, H] fp32), ``cemb`` (list of [V, H]), ``temb``,
    ``rope``, ``eps``, ``nq``, ``nkv``, optionally ``proj`` and ``proj_b``."""

    def __init__(self, weights: dict, n_positions: int = 16, cache_bf16: bool = True):
        self.w = weights
        self.n = n_positions
        self.cache_bf16 = cache_bf16

    def frame(self, x0: np.ndarray, id0: int, layer_out: list | None = None, sample: tuple | None = None):
        """Returns (codes [n], logits of positions 1..n-1); ``layer_out`` receives the residual after every layer
        at the last position. ``sample`` = (temperature, top_k, key, counter) replaces the greedy pick of position
        g >= 1 by the fused sampler's draw ``sample_draw`` with counter ``counter + g - 1`` (the sub-code draws of
        ``subtalker_dosample``, qwen3/kernels.py:671-674, one draw counter for the frame)."""
        w = self.w
        nl = len(w["layers"])
        K = np.zeros((nl, w["nkv"], self.n, HD), F32)
        V = np.zeros_like(K)
        codes, logits = [int(id0)], []
        for g in range(self.n):
            if g == 0:
                x = x0
            elif g == 1:
                x = w["temb"][codes[0]]
            else:
                x = w["cemb"][g - 2][codes[g - 1]]
            h = np.asarray(x, F32)
            if w.get("proj") is not None:
                h = gemv(h, w["proj"], w.get("proj_b"))
            for i, L in enumerate(w["layers"]):
                h = decoder_layer(h, L, w["eps"], w["rope"], K[i], V[i], g, w["nq"], w["nkv"], self.cache_bf16)
                if layer_out is not None and g == self.n - 1:
                    layer_out.append(h.copy())
            if g == 0:
                continue
            lg = rms_gemv(h, w["norm"], w["eps"], w["heads"][g - 1])
            if sample is None:
                codes.append(argmax_first(lg))
            else:
                temp, top_k, key, cnt = sample
                codes.append(sample_draw(lg, float(np.float32(1.0 / temp)), top_k, key, cnt + g - 1)[0])
            logits.append(lg)
        return codes, logits


class BatchTalkerOracle:
    """Independent talker streams stepped together, as the batched path runs them: stream b has its own caches
    ``Ks[b]`` / ``Vs[b]`` ([layers, nkv, len, 128] fp32) and position. Each step embeds every stream's token, runs
    the decoder stack with the projections of all streams as one matrix product (row b is exactly the M=1
    ``decoder_layer`` math, qwen3/kernels.py:619-627), applies the final RMSNorm inside the head projection
    (``rms_gemv`` with the final norm weight: the head GEMM of the batched path, equal in value to ``rmsnorm``
    followed by ``gemv``) and picks each stream's argmax. ``act_terms`` as ``bf16_terms`` (0: fp32 inputs)."""

    def __init__(self, weights: dict, Ks: list, Vs: list, cache_bf16: bool = True, act_terms: int = 0):
        self.w, self.Ks, self.Vs = weights, Ks, Vs
        self.cache_bf16, self.act = cache_bf16, act_terms

    def step(self, tokens, pos, layer_out: list | None = None):
        """Returns (codes [B], logits [B, V]); ``layer_out`` receives [B, H] after every layer."""
        w, B = self.w, len(tokens)
        h = np.stack([w["emb"][t] for t in tokens]).astype(F32)
        for i, L in enumerate(w["layers"]):
            qkv = rms_gemv(h, L["in_norm"], w["eps"], L["qkv"], act_bf16=self.act)
            att = np.stack([attention(qkv[b], L["qn"], L["kn"], w["eps"], w["rope"], self.Ks[b][i], self.Vs[b][i],
                                      int(pos[b]), w["nq"], w["nkv"], self.cache_bf16) for b in range(B)])
            h = gemv(att, L["o"], out=h, act_bf16=self.act)
            act = rms_gemv(h, L["post_norm"], w["eps"], L["gu"], swiglu=True, act_bf16=self.act)
            h = gemv(act, L["down"], out=h, act_bf16=self.act)
            if layer_out is not None:
                layer_out.append(h.copy())
        lg = rms_gemv(h, w["norm"], w["eps"], w["head"], act_bf16=self.act)
        return [argmax_first(lg[b]) for b in range(B)], lg

