"""Seeded synthetic Qwen3-TTS talker: random-init weights of the real architecture, shaped like the Hugging Face
modules that ``_Stack`` reads (qwen3/kernels.py:450-480), so the engine can be built without qwen-tts or a
network fetch.

Value distributions (fixed so that every run, the oracle and the GPU path see identical inputs):
  * projection weights  N(0, 0.02), drawn in float64 by numpy ``default_rng`` and stored as float32;
  * RMSNorm weights     1 + 0.1 * N(0, 1), float32 (the reference's bench uses the same form,
                        qwen3/gemv2_bench.py:109);
  * embedding table     N(0, 0.02) rounded to bf16, shape [vocab, hidden];
  * prior K/V cache     N(0, 1) rounded to bf16;
  * eps 1e-6, RoPE theta 1e6, head_dim 128, GQA with two q heads per kv head.
Each tensor has its own stream, ``SeedSequence([seed, layer + 1, tag])``, so any one layer can be regenerated
alone and the draw order never matters.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, replace
from types import SimpleNamespace

import numpy as np
import torch

_TAGS = {"q": 1, "k": 2, "v": 3, "o": 4, "gate": 5, "up": 6, "down": 7, "in_norm": 8, "post_norm": 9, "q_norm": 10,
         "k_norm": 11, "norm": 12, "head": 13, "emb": 14, "kcache": 15, "vcache": 16, "h": 17, "token": 18,
         "kvlen": 19, "prompt": 20, "proj": 21, "bias": 22}


@dataclass(frozen=True)
class TalkerShape:
    """Talker architecture. Defaults are the 0.6B talker (hidden 1024, 28 layers, 16 q / 8 kv heads,
    head_dim 128, intermediate 3072, codec vocabulary 3072)."""
    hidden: int = 1024
    n_layers: int = 28
    nq: int = 16
    nkv: int = 8
    head_dim: int = 128
    inter: int = 3072
    vocab: int = 3072
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def qkv_rows(self) -> int:
        return (self.nq + 2 * self.nkv) * self.head_dim


SHAPES = {
    "0.6b": TalkerShape(),
    "1.7b": TalkerShape(hidden=2048, inter=6144),
    "tiny": TalkerShape(hidden=512, n_layers=2, nq=4, nkv=2, inter=1024, vocab=512),
}


def shape(name: str, **over) -> TalkerShape:
    return replace(SHAPES[name], **over)


def _rng(seed: int, layer: int, tag: str) -> np.random.Generator:
    return np.random.default_rng(np.random.SeedSequence([int(seed), int(layer) + 1, _TAGS[tag]]))


def normal(seed: int, layer: int, tag: str, shp, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """float64 N(mean, std) draw, returned as float32."""
    x = _rng(seed, layer, tag).standard_normal(shp, dtype=np.float64)
    return (mean + std * x).astype(np.float32)


def bf16_values(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bf16 (nearest even) and return them as float32."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def inv_freq(s: TalkerShape) -> np.ndarray:
    """RoPE inverse frequencies computed in float32 exactly as Hugging Face's default rotary embedding does
    (``1 / theta ** (arange(0, hd, 2) / hd)``)."""
    e = torch.arange(0, s.head_dim, 2, dtype=torch.int64).to(torch.float32) / s.head_dim
    return (1.0 / (s.theta ** e)).numpy().astype(np.float32)


def layer_weights(seed: int, i: int, s: TalkerShape) -> dict:
    """fp32 weights of decoder layer ``i`` in Hugging Face layout ([out, in])."""
    H, I, hd = s.hidden, s.inter, s.head_dim
    std = 0.02
    return {
        "q": normal(seed, i, "q", (s.nq * hd, H), std), "k": normal(seed, i, "k", (s.nkv * hd, H), std),
        "v": normal(seed, i, "v", (s.nkv * hd, H), std), "o": normal(seed, i, "o", (H, s.nq * hd), std),
        "gate": normal(seed, i, "gate", (I, H), std), "up": normal(seed, i, "up", (I, H), std),
        "down": normal(seed, i, "down", (H, I), std),
        "in_norm": normal(seed, i, "in_norm", (H,), 0.1, 1.0), "post_norm": normal(seed, i, "post_norm", (H,), 0.1, 1.0),
        "q_norm": normal(seed, i, "q_norm", (hd,), 0.1, 1.0), "k_norm": normal(seed, i, "k_norm", (hd,), 0.1, 1.0),
    }


def final_weights(seed: int, s: TalkerShape) -> dict:
    L = s.n_layers
    return {"norm": normal(seed, L, "norm", (s.hidden,), 0.1, 1.0),
            "head": normal(seed, L, "head", (s.vocab, s.hidden), 0.02),
            "emb": bf16_values(normal(seed, L, "emb", (s.vocab, s.hidden), 0.02))}


def kv_prefill(seed: int, i: int, s: TalkerShape, T: int) -> tuple[np.ndarray, np.ndarray]:
    """Prior K/V for layer ``i``: [nkv, T, 128] N(0,1) rounded to bf16 (as float32 values)."""
    k = bf16_values(normal(seed, i, "kcache", (s.nkv, T, s.head_dim)))
    v = bf16_values(normal(seed, i, "vcache", (s.nkv, T, s.head_dim)))
    return k, v


def input_hidden(seed: int, s: TalkerShape) -> np.ndarray:
    """A single-layer input activation h ~ N(0,1) rounded to bf16 (as float32)."""
    return bf16_values(normal(seed, 0, "h", (s.hidden,)))


def start_token(seed: int, s: TalkerShape) -> int:
    return int(_rng(seed, 0, "token").integers(0, s.vocab))


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---------------------------------------------------------------------------------------------------------
# Hugging Face-shaped stand-ins (duck-typed attributes read by _Stack / Qwen3Kernels)
# ---------------------------------------------------------------------------------------------------------
def _p(x: np.ndarray, device, dtype=torch.float32) -> SimpleNamespace:
    return SimpleNamespace(weight=torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype), bias=None)


class _Rotary:
    def __init__(self, inv: np.ndarray, device):
        self.inv_freq = torch.from_numpy(inv).to(device)
        self.attention_scaling = 1.0


def make_talker(seed: int, s: TalkerShape, device="cpu", layers: list[dict] | None = None,
                final: dict | None = None) -> SimpleNamespace:
    """A talker object with the attributes the engine reads: ``model.layers[i].self_attn.{q,k,v,o}_proj``,
    ``q_norm``/``k_norm``, ``mlp.{gate,up,down}_proj``, ``input_layernorm``, ``post_attention_layernorm``,
    ``model.norm``, ``model.rotary_emb``, ``codec_head`` and ``get_input_embeddings()`` (bf16 table).
    ``code_predictor`` is None: the synthetic frame feeds the talker its own embedding row."""
    layers = layers if layers is not None else [layer_weights(seed, i, s) for i in range(s.n_layers)]
    final = final if final is not None else final_weights(seed, s)
    hl = []
    for w in layers:
        attn = SimpleNamespace(q_proj=_p(w["q"], device), k_proj=_p(w["k"], device), v_proj=_p(w["v"], device),
                               o_proj=_p(w["o"], device), q_norm=_p(w["q_norm"], device), k_norm=_p(w["k_norm"], device))
        mlp = SimpleNamespace(gate_proj=_p(w["gate"], device), up_proj=_p(w["up"], device), down_proj=_p(w["down"], device))
        hl.append(SimpleNamespace(self_attn=attn, mlp=mlp, input_layernorm=_p(w["in_norm"], device),
                                  post_attention_layernorm=_p(w["post_norm"], device)))
    cfg = SimpleNamespace(hidden_size=s.hidden, intermediate_size=s.inter, num_attention_heads=s.nq,
                          num_key_value_heads=s.nkv, head_dim=s.head_dim, rms_norm_eps=s.eps, rope_theta=s.theta,
                          num_hidden_layers=s.n_layers, vocab_size=s.vocab)
    model = SimpleNamespace(config=cfg, layers=hl, norm=_p(final["norm"], device),
                            rotary_emb=_Rotary(inv_freq(s), device))
    emb = SimpleNamespace(weight=torch.from_numpy(final["emb"]).to(device=device, dtype=torch.bfloat16))
    talker = SimpleNamespace(model=model, config=cfg, codec_head=_p(final["head"], device), code_predictor=None,
                             device=torch.device(device), dtype=torch.bfloat16)
    talker.get_input_embeddings = lambda: emb
    return talker


def make_tts(seed: int, s: TalkerShape, device="cpu", eos: int | None = None, **kw) -> SimpleNamespace:
    """A ``tts`` object as ``Qwen3Fast.__init__`` reads it (qwen3/fast.py:77-90): ``tts.model.talker`` and
    ``tts.model.config.talker_config`` with ``num_code_groups``, ``vocab_size`` and ``codec_eos_token_id``."""
    talker = make_talker(seed, s, device, **kw)
    # the 12 Hz codec's EOS id is 2150 in a 3072-entry vocabulary (qwen3/check_sampler.py:42)
    eos = (2150 if s.vocab > 2150 else s.vocab - 1) if eos is None else eos
    tc = SimpleNamespace(num_code_groups=1, vocab_size=s.vocab, hidden_size=s.hidden, codec_eos_token_id=eos)
    model = SimpleNamespace(talker=talker, config=SimpleNamespace(talker_config=tc))
    return SimpleNamespace(model=model)


# ---------------------------------------------------------------------------------------------------------
# code predictor (qwen3/kernels.py:516-523: cp.model, cp.lm_head[g], cp.get_input_embeddings()[g],
# cp.small_to_mtp_projection)
# ---------------------------------------------------------------------------------------------------------
CP_LAYER0, CP_FINAL, CP_HEAD0, CP_EMB0, CP_TALKER_EMB, CP_FRAME0, CP_PROJ = 100, 150, 200, 300, 400, 500, 600


def cp_weights(seed: int, s: TalkerShape, n_positions: int = 16, talker_vocab: int = 3072,
               in_hidden: int | None = None) -> dict:
    """fp32 weights of a code predictor with ``s.n_layers`` layers: its layers, final norm, heads 1..n-1
    ([vocab, hidden] each, head g produces code g), code-embedding tables 2..n-1 ([vocab, in] bf16; table g
    embeds code g - 1) and the talker's own embedding table ([talker_vocab, in]; it embeds code 0 at position 1).
    ``in_hidden`` (the talker's width, when it differs from the code predictor's) adds the input projection
    ``proj`` ([hidden, in] N(0, 0.02)) and its bias ``proj_b`` (N(0, 0.02)), the 1.7B Qwen3-TTS's
    small_to_mtp_projection; the tables are then ``in_hidden`` wide."""
    win = in_hidden or s.hidden
    w = {
        "layers": [layer_weights(seed, CP_LAYER0 + i, s) for i in range(s.n_layers)],
        "norm": normal(seed, CP_FINAL, "norm", (s.hidden,), 0.1, 1.0),
        "heads": [normal(seed, CP_HEAD0 + g, "head", (s.vocab, s.hidden), 0.02) for g in range(1, n_positions)],
        "cemb": [bf16_values(normal(seed, CP_EMB0 + g, "emb", (s.vocab, win), 0.02)) for g in range(2, n_positions)],
        "temb": bf16_values(normal(seed, CP_TALKER_EMB, "emb", (talker_vocab, win), 0.02)),
    }
    if win != s.hidden:
        w["proj"] = normal(seed, CP_PROJ, "proj", (s.hidden, win), 0.02)
        w["proj_b"] = normal(seed, CP_PROJ, "bias", (s.hidden,), 0.02)
    return w


def cp_frame_inputs(seed: int, f: int, s: TalkerShape, talker_vocab: int = 3072,
                    in_hidden: int | None = None) -> tuple[np.ndarray, int]:
    """Inputs of code-predictor frame ``f``: the talker's last hidden state x0 ~ N(0, 1) (fp32; ``in_hidden``
    wide when given, else the code predictor's width) and code 0."""
    x0 = normal(seed, CP_FRAME0 + f, "h", (in_hidden or s.hidden,))
    return x0, int(_rng(seed, CP_FRAME0 + f, "token").integers(0, talker_vocab))


def make_code_predictor(seed: int, s: TalkerShape, device="cpu", n_positions: int = 16, w: dict | None = None,
                        in_hidden: int | None = None):
    """(cp, talker embedding) with the attributes the engine reads: ``cp.model`` (layers, norm, rotary_emb,
    config), ``cp.lm_head`` (n - 1 heads), ``cp.get_input_embeddings()`` (n - 1 tables: entry g - 1 embeds
    code g; the last one is only used by the talker's input), ``cp.small_to_mtp_projection`` (identity when the
    talker and the code predictor are equally wide, else a ``torch.nn.Linear`` with bias, from the weights'
    ``proj`` / ``proj_b``; ``in_hidden`` is the talker's width) and ``cp.config.vocab_size``."""
    w = w if w is not None else cp_weights(seed, s, n_positions, in_hidden=in_hidden)
    win = w["temb"].shape[1]
    base = make_talker(seed, s, device, layers=w["layers"],
                       final={"norm": w["norm"], "head": w["heads"][0], "emb": w["temb"]})
    cemb = [SimpleNamespace(weight=torch.from_numpy(t).to(device=device, dtype=torch.bfloat16)) for t in w["cemb"]]
    # the talker's input also embeds the last code: one more table, unused by the code predictor itself
    cemb.append(SimpleNamespace(weight=torch.zeros((s.vocab, win), dtype=torch.bfloat16, device=device)))
    proj = torch.nn.Identity()
    if "proj" in w:
        proj = torch.nn.Linear(win, s.hidden, bias=True)
        with torch.no_grad():
            proj.weight.copy_(torch.from_numpy(w["proj"]))
            proj.bias.copy_(torch.from_numpy(w["proj_b"]))
        proj = proj.to(device)
    cp = SimpleNamespace(model=base.model, lm_head=[_p(h, device) for h in w["heads"]],
                         small_to_mtp_projection=proj, config=SimpleNamespace(vocab_size=s.vocab))
    cp.get_input_embeddings = lambda: cemb
    temb = torch.from_numpy(w["temb"]).to(device=device, dtype=torch.bfloat16)
    return cp, temb


def make_tts_with_cp(seed: int, s: TalkerShape, cp_shape: TalkerShape, device="cpu", n_groups: int = 16):
    """A ``tts`` whose talker carries a code predictor of ``cp_shape`` (n_groups - 1 heads and code tables; its
    position 1 embeds code 0 with the talker's own table), as the reference reads a real Qwen3-TTS model
    (qwen3/kernels.py:514-523). Returns (tts, pad row): the pad row is the bf16 ``tts_pad_embed`` added to every
    talker input, N(0, 0.02)."""
    tts = make_tts(seed, s, device=device)
    w = cp_weights(seed, cp_shape, n_groups, talker_vocab=s.vocab,
                   in_hidden=s.hidden if s.hidden != cp_shape.hidden else None)
    w["temb"] = final_weights(seed, s)["emb"]
    cp, _ = make_code_predictor(seed, cp_shape, device=device, n_positions=n_groups, w=w)
    tts.model.talker.code_predictor = cp
    tts.model.config.talker_config.num_code_groups = n_groups
    pad = bf16_values(normal(seed, CP_FRAME0 - 1, "emb", (s.hidden,), 0.02))
    return tts, pad


# ---------------------------------------------------------------------------------------------------------
# named workloads
# ---------------------------------------------------------------------------------------------------------
WORKLOADS = {
    # single 0.6B-shaped decoder layer, one token, 256 prior positions (T = 257)
    "layer06b": dict(shape="0.6b", n_layers=1, kv=256),
    # 0.6B-shaped talker: 28 layers + final norm + 3072-way codec head, KV 512, 64 greedy frames
    "talker06b": dict(shape="0.6b", n_layers=28, kv=512, frames=64),
    # 1.7B-shaped talker: hidden 2048, intermediate 6144, KV 1024, 64 greedy frames
    "talker17b": dict(shape="1.7b", n_layers=28, kv=1024, frames=64),
    # tiny two-layer model for quick checks
    "tiny": dict(shape="tiny", n_layers=2, kv=24, frames=8),
    # two 0.6B-shaped layers (the persistent frame kernel needs the real head counts)
    "small06b": dict(shape="0.6b", n_layers=2, kv=40, frames=8),
    # two 1.7B-shaped layers (the frame kernel's 8-compute-wave variant)
    "small17b": dict(shape="1.7b", n_layers=2, kv=40, frames=8),
    # code predictor: 5 layers of the 0.6B shape, 2048-way heads, 16 positions (KV 1 -> 16) per frame, greedy
    # sub-codes; a step is `frames` code-predictor frames with different (x0, code 0)
    "cp06b": dict(shape="0.6b", n_layers=5, vocab=2048, kv=0, positions=16, frames=8),
    # the 1.7B Qwen3-TTS code predictor: the same 1024-wide stack behind a projection from the talker's 2048-wide
    # hidden state and embedding rows (small_to_mtp_projection, with bias)
    "cp17b": dict(shape="0.6b", n_layers=5, vocab=2048, kv=0, positions=16, frames=8, in_hidden=2048),
    # the whole Qwen3-TTS frame: the 0.6B talker (KV 512) fed by a 5-layer code predictor (16 code groups),
    # 64 greedy frames
    "frame06b": dict(shape="0.6b", n_layers=28, kv=512, frames=64, cp="cp06b"),
    # the whole 1.7B Qwen3-TTS frame: the 1.7B talker (KV 1024) fed by the projected code predictor
    "frame17b": dict(shape="1.7b", n_layers=28, kv=1024, frames=64, cp="cp17b"),
    # the same with a two-layer talker, for quick checks
    "frame17small": dict(shape="1.7b", n_layers=2, kv=40, frames=8, cp="cp17b"),
    # 16 concurrent 1.7B-shaped streams, prior KV lengths uniform in [64, 2048], 32 greedy frames
    "batch17b": dict(shape="1.7b", n_layers=28, kv=0, batch=16, kv_lo=64, kv_hi=2048, frames=32),
    # the same with two layers and five streams, for quick checks
    "batchsmall": dict(shape="1.7b", n_layers=2, kv=0, batch=5, kv_lo=8, kv_hi=200, frames=6),
}


def workload_shape(name: str) -> TalkerShape:
    w = WORKLOADS[name]
    return shape(w["shape"], n_layers=w["n_layers"], **({"vocab": w["vocab"]} if "vocab" in w else {}))


# ---------------------------------------------------------------------------------------------------------
# batched streams
# ---------------------------------------------------------------------------------------------------------
def batch_lengths(seed: int, name: str) -> list[int]:
    """Prior KV length of every stream of a batched workload, uniform in [kv_lo, kv_hi]."""
    w = WORKLOADS[name]
    return [int(t) for t in _rng(seed, 0, "kvlen").integers(w["kv_lo"], w["kv_hi"] + 1, w["batch"])]


def batch_tokens(seed: int, name: str) -> list[int]:
    """First input token of every stream of a batched workload."""
    w = WORKLOADS[name]
    return [int(t) for t in _rng(seed, 1, "token").integers(0, workload_shape(name).vocab, w["batch"])]


def batch_prefill(seed: int, i: int, b: int, s: TalkerShape, T: int) -> tuple[np.ndarray, np.ndarray]:
    """Prior K/V of layer ``i`` of stream ``b``: [nkv, T, 128] N(0, 1) drawn in float32 and rounded to bf16."""
    out = []
    for tag in ("kcache", "vcache"):
        g = np.random.default_rng(np.random.SeedSequence([int(seed), int(i) + 1, _TAGS[tag], 1000 + int(b)]))
        out.append(bf16_values(g.standard_normal((s.nkv, T, s.head_dim), dtype=np.float32)))
    return out[0], out[1]


def batch_max_len(name: str, frames: int | None = None) -> int:
    w = WORKLOADS[name]
    return w["kv_hi"] + (w["frames"] if frames is None else frames) + 1


def make_frame_engine(name: str = "frame06b", seed: int = 0, device="cuda", frame_kernel: bool | None = None,
                      sampled: bool = False, wd: str = "i8row"):
    """A Qwen3Kernels engine over the seeded synthetic talker with a code predictor (workload ``name``), prior cache
    loaded, state at position ``kv``. Greedy without the processor, or with ``sampled`` the reference's default
    settings (``Sampling()``: temperature 0.9, top_k 50, repetition penalty 1.05, 2 codes before EOS, sub-codes at
    0.9 / 50, the last 1024 ids suppressed); ``wd`` the weight format. Returns (engine, start token, kw) where kw
    holds the prefill results
    ``generate_codes`` takes (``prefill_len``, ``first_token``, ``last_hidden``, ``tts_pad_embed``) and the
    sampling settings."""
    from .fast import Sampling
    from .kernels import Qwen3Kernels

    w = WORKLOADS[name]
    s = workload_shape(name)
    cs = workload_shape(w["cp"])
    tts, pad = make_tts_with_cp(seed, s, cs, device=device)
    smp = Sampling(max_new_tokens=4096) if sampled else Sampling.greedy(processor=False, max_new_tokens=4096)
    eng = Qwen3Kernels(tts, smp, max_cache=w["kv"] + w["frames"] + 1, wd=wd, sampler="fused",
                       suppress_tail=1024 if sampled else 0, frame_kernel=frame_kernel)
    eng.talker = None
    del tts
    for i in range(s.n_layers):
        k, v = kv_prefill(seed, i, s, w["kv"])
        eng.kc[i, :, :w["kv"]].copy_(torch.from_numpy(k).to(eng.kc.dtype))
        eng.vc[i, :, :w["kv"]].copy_(torch.from_numpy(v).to(eng.vc.dtype))
    tok = start_token(seed, s)
    x0, _ = cp_frame_inputs(seed, 0, s)
    kw = {"prefill_len": w["kv"], "first_token": tok, "last_hidden": torch.from_numpy(x0), "tts_pad_embed": torch.from_numpy(pad),
          "do_sample": smp.do_sample, "temperature": smp.temperature, "top_k": smp.top_k,
          "repetition_penalty": smp.repetition_penalty, "min_new_tokens": smp.min_new_tokens, "max_new_tokens": 4096,
          "subtalker_dosample": smp.sub_do_sample, "subtalker_temperature": smp.sub_temperature,
          "subtalker_top_k": smp.sub_top_k}
    eng._start(kw)
    return eng, tok, kw


def make_batch_engine(name: str, seed: int = 0, device="cuda", frames: int | None = None, progress=None):
    """A BatchedTalker over the seeded synthetic talker of a batched workload, every stream's prior cache loaded
    and the first tokens embedded. ``frames``: how many steps the cache must leave room for (default the
    workload's); ``progress(message)`` is called after each stage. Returns (engine, lengths, tokens)."""
    from .batch import BatchedTalker

    w = WORKLOADS[name]
    s = workload_shape(name)
    frames = w["frames"] if frames is None else frames
    tts = make_tts(seed, s, device=device)
    if progress:
        progress("weights generated")
    eng = BatchedTalker(tts.model.talker, w["batch"], batch_max_len(name, frames), max_frames=max(frames, 1),
                        device=device)
    del tts
    if progress:
        progress("weights packed")
    T = batch_lengths(seed, name)
    for b in range(w["batch"]):
        for i in range(s.n_layers):
            k, v = batch_prefill(seed, i, b, s, T[b])
            eng.kc[i, b, :, :T[b]].copy_(torch.from_numpy(k).to(torch.bfloat16))
            eng.vc[i, b, :, :T[b]].copy_(torch.from_numpy(v).to(torch.bfloat16))
        if progress:
            progress(f"stream {b} prefilled ({T[b]} positions)")
    tok = batch_tokens(seed, name)
    eng.reset(T, tok)
    return eng, T, tok


def make_engine(name: str, seed: int = 0, wd: str = "i8row", device="cuda", graphs: bool = True,
                max_cache: int | None = None, frames: int | None = None, frame_kernel: bool | None = False,
                sampling=None, suppress_tail: int = 0):
    """Builds a Qwen3Kernels engine over the seeded synthetic talker of workload ``name`` with the prior KV
    cache loaded and the frame state set at position ``kv``. By default greedy decoding without the processor
    (plain argmax over the whole codec vocabulary); ``sampling`` (a ``Sampling``) overrides. Returns
    (engine, start token)."""
    from .fast import Sampling
    from .kernels import Qwen3Kernels

    w = WORKLOADS[name]
    s = workload_shape(name)
    frames = w.get("frames", 1) if frames is None else frames
    max_cache = max_cache or (w["kv"] + frames + 1)
    tts = make_tts(seed, s, device=device)
    eng = Qwen3Kernels(tts, sampling or Sampling.greedy(processor=False), max_cache=max_cache, wd=wd, graphs=graphs,
                       sampler="fused", suppress_tail=suppress_tail, frame_kernel=frame_kernel)
    tts.model.talker = None  # the fp32 source weights are no longer needed once packed
    eng.talker = None
    del tts
    dt = eng.kc.dtype
    for i in range(s.n_layers):
        k, v = kv_prefill(seed, i, s, w["kv"])
        eng.kc[i, :, :w["kv"]].copy_(torch.from_numpy(k).to(dt))
        eng.vc[i, :, :w["kv"]].copy_(torch.from_numpy(v).to(dt))
    tok = start_token(seed, s)
    eng.reset(w["kv"], tok)
    return eng, tok


def hf_talker_model(seed: int, s: TalkerShape, device="cpu", attn: str = "sdpa"):
    """transformers' Qwen3Model (fp32; SDPA attention as the reference loads the talker, qwen3/serve.py:89, or
    ``attn``) holding the seeded synthetic weights of shape ``s``: a runnable stand-in for
    ``tts.model.talker.model``, for prompts given as ``inputs_embeds``."""
    from transformers import Qwen3Config, Qwen3Model

    cfg = Qwen3Config(hidden_size=s.hidden, intermediate_size=s.inter, num_attention_heads=s.nq,
                      num_key_value_heads=s.nkv, head_dim=s.head_dim, rms_norm_eps=s.eps, num_hidden_layers=s.n_layers,
                      vocab_size=s.vocab, rope_parameters={"rope_type": "default", "rope_theta": s.theta},
                      attention_bias=False)
    cfg._attn_implementation = attn
    model = Qwen3Model(cfg).float().eval()
    final = final_weights(seed, s)
    with torch.no_grad():
        for i, layer in enumerate(model.layers):
            w = layer_weights(seed, i, s)
            a, m = layer.self_attn, layer.mlp
            for mod, key in ((a.q_proj, "q"), (a.k_proj, "k"), (a.v_proj, "v"), (a.o_proj, "o"), (m.gate_proj, "gate"),
                             (m.up_proj, "up"), (m.down_proj, "down"), (a.q_norm, "q_norm"), (a.k_norm, "k_norm"),
                             (layer.input_layernorm, "in_norm"), (layer.post_attention_layernorm, "post_norm")):
                mod.weight.copy_(torch.from_numpy(w[key]))
        model.norm.weight.copy_(torch.from_numpy(final["norm"]))
        model.embed_tokens.weight.copy_(torch.from_numpy(final["emb"]))
    return model.to(device)


def prompt_embeds(seed: int, s: TalkerShape, L: int) -> np.ndarray:
    """A prompt of L input rows (1, L, H): N(0, 0.02) rounded to bf16 (as float32), like embedding rows."""
    return bf16_values(normal(seed, 0, "prompt", (1, L, s.hidden), 0.02))


def make_prefill_engine(name: str, seed: int = 0, L: int = 24, frames: int = 8, device="cuda",
                        frame_kernel: bool | None = False, cp: str | None = None):
    """A Qwen3Kernels engine whose talker modules are runnable (``hf_talker_model``), an empty cache of
    L + frames + 1 positions and greedy settings without the processor; with ``cp`` (a code-predictor workload
    name) the talker carries that code predictor and the pad row. The prompt goes in through
    ``generate_codes({"inputs_embeds": ...})``. Returns (engine, generate kwargs)."""
    from .fast import Sampling
    from .kernels import Qwen3Kernels

    s = workload_shape(name)
    pad = None
    if cp is None:
        tts = make_tts(seed, s, device=device)
    else:
        tts, pad = make_tts_with_cp(seed, s, workload_shape(cp), device=device)
    tts.model.talker.model = hf_talker_model(seed, s, device)
    smp = Sampling.greedy(processor=False)
    eng = Qwen3Kernels(tts, smp, max_cache=L + frames + 1, wd="i8row", graphs=True, sampler="fused",
                       suppress_tail=0, frame_kernel=frame_kernel)
    kw = {"inputs_embeds": torch.from_numpy(prompt_embeds(seed, s, L)).to(device), "do_sample": False,
          "subtalker_dosample": False, "max_new_tokens": smp.max_new_tokens, "repetition_penalty": 1.0,
          "min_new_tokens": 0}
    if pad is not None:
        kw["tts_pad_embed"] = torch.from_numpy(pad).to(device)
    return eng, kw


def make_cp_engine(name: str = "cp06b", seed: int = 0, device="cuda", keep_layers: bool = True,
                   pair: bool | None = None, wd: str = "i8row", positions: int | None = None):
    """A CodePredictor over the seeded synthetic code predictor of workload ``name`` (one frame per run);
    ``keep_layers``, ``pair`` and ``wd`` as CodePredictor's (layer weights loaded cacheable, positions 0 and 1
    paired unless the code predictor is projected, i8row: the defaults); ``positions`` overrides the workload's
    count of positions."""
    from .kernels import CodePredictor

    n = positions or WORKLOADS[name]["positions"]
    s = workload_shape(name)
    cp, temb = make_code_predictor(seed, s, device=device, n_positions=n, in_hidden=WORKLOADS[name].get("in_hidden"))
    return CodePredictor(cp, temb, n_positions=n, wd=wd, device=device, keep_layers=keep_layers, pair=pair)


# ---------------------------------------------------------------------------------------------------------
# an HF-shaped stand-in for the qwen-tts object (prompt interception, prefill, speech-tokenizer decode)
# ---------------------------------------------------------------------------------------------------------
class _ToyCodecDecoder(torch.nn.Module):
    """A causal stand-in for the speech tokenizer's decoder: codes (1, G, F) int64 -> waveform (1, 1, F * up). Each
    frame's samples come from the sum of its G code embeddings plus half the previous frame's (one frame of left
    context), so a prefix of frames decodes the same whatever follows, as the real causal decoder does."""

    def __init__(self, seed: int, groups: int, vocab: int, up: int):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.tables = torch.nn.Parameter(torch.randn(groups, vocab, up, generator=g) * 0.1, requires_grad=False)
        self.total_upsample = up

    def forward(self, codes: torch.Tensor) -> torch.Tensor:
        G = self.tables.shape[0]
        x = sum(self.tables[g][codes[0, g]] for g in range(G))  # (F, up)
        prev = torch.cat([torch.zeros_like(x[:1]), x[:-1]], dim=0)
        return torch.tanh(x + 0.5 * prev).reshape(1, 1, -1)


def make_hf_tts(name: str = "small06b", seed: int = 0, device="cpu", up: int = 40):
    """A ``tts`` object with what the prompt, prefill and decode paths of the engine read from qwen-tts
    (qwen3/fast.py:127-147, 251-368): ``generate_custom_voice`` builds a prompt from the text (rows N(0, 0.02) from
    a seed of the text, length 6 + len(text)) and hands it to ``model.talker.generate`` with the official keyword
    arguments; ``model.talker.model`` is a runnable transformers Qwen3Model (fp32) holding the synthetic weights;
    ``model.speech_tokenizer`` decodes codes with a small causal decoder (``decode`` and ``model.decoder``,
    ``total_upsample``, ``decode_upsample_rate``, ``get_output_sample_rate``). Greedy settings by default."""
    s = workload_shape(name)
    tts = make_tts(seed, s, device=device)
    talker = tts.model.talker
    talker.model = hf_talker_model(seed, s, device)
    talker.dtype = torch.float32

    def talker_generate(**kw):  # the official generation; the engine intercepts this call and never runs it
        raise RuntimeError("the stand-in talker cannot generate")

    talker.generate = talker_generate
    pad = torch.from_numpy(bf16_values(normal(seed, 0, "prompt", (1, 1, s.hidden), 0.02))).to(device)

    def generate_custom_voice(text: str, speaker: str, language: str, do_sample: bool = False, top_k: int = 50,
                              top_p: float = 1.0, temperature: float = 0.9, repetition_penalty: float = 1.0,
                              min_new_tokens: int = 0, max_new_tokens: int = 2048, subtalker_dosample: bool = False,
                              subtalker_top_k: int = 50, subtalker_top_p: float = 1.0,
                              subtalker_temperature: float = 0.9):
        L = 6 + len(text)
        h = int.from_bytes(hashlib.sha256(f"{speaker}|{language}|{text}".encode()).digest()[:4], "little")
        rows = bf16_values(np.random.default_rng(h).standard_normal((1, L, s.hidden)) * 0.02)
        emb = torch.from_numpy(rows.astype(np.float32)).to(device)
        return talker.generate(inputs_embeds=emb, attention_mask=torch.ones((1, L), dtype=torch.long, device=device),
                               trailing_text_hidden=pad.clone(), tts_pad_embed=pad.clone(), do_sample=do_sample,
                               top_k=top_k, top_p=top_p, temperature=temperature,
                               repetition_penalty=repetition_penalty, min_new_tokens=min_new_tokens,
                               max_new_tokens=max_new_tokens, subtalker_dosample=subtalker_dosample,
                               subtalker_top_k=subtalker_top_k, subtalker_top_p=subtalker_top_p,
                               subtalker_temperature=subtalker_temperature)

    groups = int(tts.model.config.talker_config.num_code_groups)
    decoder = _ToyCodecDecoder(seed, groups, s.vocab, up).to(device)

    def tok_decode(items):
        wavs = []
        with torch.inference_mode():
            for it in items:
                c = torch.clamp(torch.as_tensor(it["audio_codes"]), min=0).t().unsqueeze(0).to(device)
                wavs.append(decoder(c).reshape(-1).float().cpu().numpy())
        return wavs, 24000

    tok_model = SimpleNamespace(decoder=decoder, decode_upsample_rate=up, get_output_sample_rate=lambda: 24000)
    tts.model.speech_tokenizer = SimpleNamespace(model=tok_model, decode=tok_decode)
    tts.generate_custom_voice = generate_custom_voice
    tts.get_supported_speakers = lambda: ["vivian"]
    return tts
