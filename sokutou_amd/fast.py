"""Frame-loop orchestration shared by the engines: sampling settings, the torch sampling path, state buffers,
HIP-graph capture of one frame and the host frame loop.

Mirrors the call surface of the reference's qwen3/fast.py (``Sampling`` 29-51, ``_multinomial`` 54-58,
``_sample`` 61-71, ``Qwen3Fast`` 74-388). The reference drives Hugging Face modules from Python for the
frame; here the frame body is always supplied by a subclass (``Qwen3Kernels``), and the HF-module paths
(prompt interception, prefill graphs, codec decode) are left to the real-model integration.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import torch


@dataclass
class Sampling:
    """Generation settings the talker is driven with (field names and defaults as qwen3/fast.py:29-41)."""
    do_sample: bool = True
    temperature: float = 0.9
    top_k: int = 50
    repetition_penalty: float = 1.05
    min_new_tokens: int = 2
    max_new_tokens: int = 2048
    sub_do_sample: bool = True
    sub_temperature: float = 0.9
    sub_top_k: int = 50

    @classmethod
    def from_kwargs(cls, kw: dict) -> "Sampling":
        """Builds the settings from intercepted ``generate`` kwargs; top_p other than 1.0 is refused
        (qwen3/fast.py:42-51)."""
        for k in ("top_p", "subtalker_top_p"):
            if kw.get(k, 1.0) != 1.0:
                raise ValueError(f"{k}={kw[k]} is not supported (only 1.0)")
        d = cls()
        return cls(do_sample=bool(kw.get("do_sample", d.do_sample)), temperature=float(kw.get("temperature", d.temperature)),
                   top_k=int(kw.get("top_k", d.top_k)),
                   repetition_penalty=float(kw.get("repetition_penalty", d.repetition_penalty)),
                   min_new_tokens=int(kw.get("min_new_tokens", d.min_new_tokens)),
                   max_new_tokens=int(kw.get("max_new_tokens", d.max_new_tokens)),
                   sub_do_sample=bool(kw.get("subtalker_dosample", d.sub_do_sample)),
                   sub_temperature=float(kw.get("subtalker_temperature", d.sub_temperature)),
                   sub_top_k=int(kw.get("subtalker_top_k", d.sub_top_k)))

    @classmethod
    def greedy(cls, processor: bool = True, max_new_tokens: int = 2048) -> "Sampling":
        """Greedy decoding; with ``processor=False`` the repetition penalty and the min-new-tokens EOS block are
        neutral (penalty 1.0, min_new 0)."""
        return cls(do_sample=False, sub_do_sample=False, max_new_tokens=max_new_tokens,
                   repetition_penalty=1.05 if processor else 1.0, min_new_tokens=2 if processor else 0)


def _multinomial(probs: torch.Tensor) -> torch.Tensor:
    """One draw of ``torch.multinomial(probs, 1)`` without its host-side check, as argmax(p / q) with
    q ~ Exp(1) (the single-sample shortcut ATen uses), so it can be graph-captured (qwen3/fast.py:54-58)."""
    q = torch.empty_like(probs).exponential_(1)
    return torch.argmax(probs / q, dim=-1, keepdim=True)


def _sample(scores: torch.Tensor, do_sample: bool, temperature: float, top_k: int) -> torch.Tensor:
    """Warpers + softmax + draw, or argmax when not sampling; scores fp32 (1, V) (qwen3/fast.py:61-71)."""
    if not do_sample:
        return torch.argmax(scores, dim=-1, keepdim=True)
    if temperature != 1.0:
        scores = scores / temperature
    if top_k:
        kth = torch.topk(scores, min(top_k, scores.shape[-1]))[0][..., -1, None]
        scores = scores.masked_fill(scores < kth, -float("inf"))
    return _multinomial(torch.softmax(scores, dim=-1))


class Qwen3Fast:
    """State buffers, capture and the host frame loop (qwen3/fast.py:74-249). ``_frame`` is supplied by the
    subclass; it reads ``id0``/``pos`` from device memory, so one captured graph is replayed for every frame."""

    def __init__(self, tts, sampling: Sampling | None = None, max_cache: int = 1024, compile: bool = False,
                 graphs: bool = True, suppress_tail: int = 1024):
        if compile:
            raise ValueError("compile=True (torch.compile of the HF frame) is not provided by this engine")
        self.tts = tts
        self.model = tts.model
        self.talker = self.model.talker
        self.cp = getattr(self.talker, "code_predictor", None)
        cfg = self.model.config.talker_config
        self.cfg = cfg
        self.s = sampling or Sampling()
        self.G = int(cfg.num_code_groups)
        self.V = int(cfg.vocab_size)
        self.eos = int(cfg.codec_eos_token_id)
        self.max_cache = int(max_cache)
        dev = torch.device(getattr(self.talker, "device", "cuda"))
        self.device, self.dtype = dev, getattr(self.talker, "dtype", torch.bfloat16)
        # ids suppressed for the first code: the last `suppress_tail` ids except EOS (qwen3/fast.py:93-97)
        sup = torch.zeros((1, self.V), dtype=torch.bool, device=dev)
        if suppress_tail:
            sup[:, self.V - suppress_tail:] = True
            sup[:, self.eos] = False
        self.suppress = sup
        self.suppress_tail = suppress_tail
        self.id0 = torch.zeros((1, 1), dtype=torch.long, device=dev)
        self.pos = torch.zeros((1,), dtype=torch.long, device=dev)
        self.seen = torch.zeros((1, self.V), dtype=torch.bool, device=dev)
        self.ngen = torch.zeros((1,), dtype=torch.long, device=dev)
        self.codes = torch.zeros((1, self.G), dtype=torch.long, device=dev)
        self.next_id0 = torch.zeros((1, 1), dtype=torch.long, device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.stats: dict = {}
        self.graphs = graphs and dev.type == "cuda"

    # --- sampling on the torch path -----------------------------------------------------------------------
    def _process(self, scores: torch.Tensor) -> torch.Tensor:
        """Talker processor on fp32 (1, V) logits: repetition penalty on seen ids, suppressed ids, EOS blocked
        until ``min_new_tokens`` codes exist (qwen3/fast.py:154-166)."""
        p = self.s.repetition_penalty
        if p != 1.0:
            scores = torch.where(self.seen, torch.where(scores < 0, scores * p, scores / p), scores)
        scores = scores.masked_fill(self.suppress, -float("inf"))
        block = (self.ngen < self.s.min_new_tokens).view(1, 1)
        eos_col = scores[:, self.eos:self.eos + 1]
        eos_col = torch.where(block, torch.full_like(eos_col, -float("inf")), eos_col)
        return torch.cat([scores[:, :self.eos], eos_col, scores[:, self.eos + 1:]], dim=-1)

    def _frame(self) -> None:
        raise NotImplementedError

    # Frames between reads of the kernels' device error words in generate_codes (and once after the loop). A kernel
    # that fails leaves the frame state alone, so the loop would replay the same frame; the check bounds that to
    # this many frames, and the codes are never returned.
    ERROR_CHECK_EVERY = 16

    def _check_errors(self) -> None:
        """Raises RuntimeError if a kernel of the frame reported an error on the device; subclasses override."""

    # --- capture ------------------------------------------------------------------------------------------
    def _state(self):
        return (self.id0, self.pos, self.seen, self.ngen)

    def capture(self) -> float:
        """Records one frame as a HIP graph: three warm-up frames on a side stream, then capture, then the frame
        state is restored so capturing has no visible effect (qwen3/fast.py:201-218)."""
        t0 = time.perf_counter()
        saved = [t.clone() for t in self._state()]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(3):
                self._frame()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g), torch.no_grad():
            self._frame()
        for t, v in zip(self._state(), saved):
            t.copy_(v)
        self.graph = g
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    # --- host frame loop ----------------------------------------------------------------------------------
    def _start(self, kw: dict) -> int:
        """Sets the frame state after the prompt; returns the prompt length L. Subclasses override."""
        raise NotImplementedError

    @torch.no_grad()
    def generate_codes(self, kw: dict, max_frames: int | None = None) -> torch.Tensor:
        """Frames until EOS or a cap: one graph replay (or one eager frame) per frame and one host read of the
        next id (qwen3/fast.py:221-249). Returns the codes (frames, G) and fills ``stats``."""
        step = self.graph.replay if self.graph is not None else self._frame
        if Sampling.from_kwargs(kw) != self.s:
            raise ValueError(f"settings differ from the captured ones {self.s}: {Sampling.from_kwargs(kw)}")
        L = self._start(kw)
        limit = min(self.s.max_new_tokens - 1, self.max_cache - L)
        if limit <= 0:
            raise ValueError(f"prompt too long ({L} tokens, cache {self.max_cache})")
        cap = limit if max_frames is None else min(limit, max_frames)
        frames = []
        nid = int(self.id0.item())
        while nid != self.eos and len(frames) < cap:
            step()
            frames.append(self.codes.clone())
            nid = int(self.next_id0.item())
            if len(frames) % self.ERROR_CHECK_EVERY == 0:
                self._check_errors()
        self._check_errors()
        self.stats["prompt_tokens"] = L
        self.stats["stopped"] = nid == self.eos
        self.stats["cache_limited"] = nid != self.eos and len(frames) == limit and limit < self.s.max_new_tokens - 1
        self.stats["frame_limited"] = nid != self.eos and cap < limit and len(frames) == cap
        return torch.cat(frames, dim=0) if frames else torch.zeros((0, self.G), dtype=torch.long, device=self.device)
