"""Frame-loop orchestration shared by the engines: sampling settings, the torch sampling path, state buffers,
HIP-graph capture of one frame and the host frame loop.

Mirrors the call surface of the reference's qwen3/fast.py (``Sampling`` 29-51, ``_multinomial`` 54-58,
``_sample`` 61-71, ``Qwen3Fast`` 74-388): prompt interception from the official ``generate_custom_voice``, the
prompt prefill (one captured graph per prompt length), the frame loop, and the speech-tokenizer decode (one captured
graph per length bucket). The frame body and the prefill body are supplied by a subclass (``Qwen3Kernels``).
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


class _Captured(Exception):
    """Carries the keyword arguments the official pipeline passed to the talker's ``generate``."""

    def __init__(self, kwargs: dict):
        super().__init__("talker.generate intercepted")
        self.kwargs = kwargs


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
        self.tcache = None  # the talker's KV cache as a transformers cache object (set by an engine that has one)
        self._pf: dict = {}   # prompt length -> (graph, input buffer, positions)
        self._dec: dict = {}  # decode bucket -> (graph, code buffer, output)
        self._pool = torch.cuda.graph_pool_handle() if self.graphs else None

    # --- prompt ---------------------------------------------------------------------------------------------
    def prompt(self, text: str, speaker: str, language: str, **gen) -> dict:
        """Runs the official ``tts.generate_custom_voice`` up to the point where it hands the prompt to the
        talker's ``generate``, and returns that call's keyword arguments (``inputs_embeds``, ``tts_pad_embed``, the
        sampling settings ...). ``gen`` are generate_custom_voice's generation arguments. Only prompts with the text
        inside (every step adds ``tts_pad_embed``) and one unpadded sentence are accepted, as in qwen3/fast.py:127-147."""
        talker = self.talker
        had_own = "generate" in vars(talker)
        own = vars(talker).get("generate")

        def intercept(*args, **kw):
            raise _Captured(kw)

        talker.generate = intercept
        kw = None
        try:
            self.tts.generate_custom_voice(text=text, speaker=speaker, language=language, **gen)
        except _Captured as c:
            kw = c.kwargs
        finally:
            if had_own:
                talker.generate = own
            else:
                del talker.generate
        if kw is None:
            raise RuntimeError("generate_custom_voice returned without calling the talker's generate")
        tth, pad = kw["trailing_text_hidden"], kw["tts_pad_embed"]
        if tth.shape[1] != 1 or not torch.equal(tth, pad):
            raise ValueError("only prompts with the whole text inside (non-streaming mode) are supported")
        if not bool(kw["attention_mask"].all()):
            raise ValueError("only one unpadded sentence per prompt is supported")
        return kw

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

    # --- prompt prefill --------------------------------------------------------------------------------------
    def _prefill_body(self, embeds: torch.Tensor, cpos: torch.Tensor) -> None:
        """The prompt (1, L, H) through the talker into the cache, the first code and the frame state; supplied by
        the engine. Must be graph-capturable (no host reads)."""
        raise NotImplementedError

    def _prompt_dtype(self) -> torch.dtype:
        """Element type of the prompt rows the prefill takes (the talker's)."""
        return self.dtype

    @torch.no_grad()
    def _prefill(self, embeds: torch.Tensor) -> None:
        """Runs ``_prefill_body``: eagerly without graphs, else by replaying the graph recorded for this prompt length
        (recorded on first use; ``warm_prefill`` records ahead of time)."""
        L = int(embeds.shape[1])
        if not self.graphs:
            self._prefill_body(embeds, torch.arange(L, device=self.device))
            return
        if L not in self._pf:
            self._pf[L] = self._capture_prefill(L)
        g, buf, _ = self._pf[L]
        buf.copy_(embeds)
        g.replay()

    def _capture_prefill(self, L: int):
        """Records the prefill of an L-row prompt: two warm-up runs on a side stream, then the capture into the
        engine's graph pool. The RNG state is put back afterwards, so recording draws nothing a later run sees."""
        t0 = time.perf_counter()
        buf = torch.zeros((1, L, int(self.cfg.hidden_size)), dtype=self._prompt_dtype(), device=self.device)
        cpos = torch.arange(L, device=self.device)
        rng = torch.cuda.get_rng_state(self.device)
        saved = [t.clone() for t in self._state()]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(2):
                self._prefill_body(buf, cpos)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=self._pool), torch.no_grad():
            self._prefill_body(buf, cpos)
        torch.cuda.synchronize()
        for t, v in zip(self._state(), saved):
            t.copy_(v)
        torch.cuda.set_rng_state(rng, self.device)
        self.stats["prefill_capture_sec"] = self.stats.get("prefill_capture_sec", 0.0) + time.perf_counter() - t0
        return g, buf, cpos

    def warm_prefill(self, lengths) -> float:
        """Records the prefill graphs of the given prompt lengths ahead of time; returns the seconds spent
        (qwen3/fast.py:294-300)."""
        t0 = time.perf_counter()
        if self.graphs:
            for L in lengths:
                if int(L) not in self._pf:
                    self._pf[int(L)] = self._capture_prefill(int(L))
        return time.perf_counter() - t0

    # --- speech-tokenizer decode -----------------------------------------------------------------------------
    # frame counts the decode graphs are recorded for (a segment is padded up to the next one), as the reference
    DEC_BUCKETS = (16, 24, 32, 40, 48, 56, 64, 72, 80, 96, 112, 128, 160, 192, 224, 256, 300, 325)
    DEC_CHUNK, DEC_CONTEXT = 300, 25  # the official chunked decode: 300 frames, 25 frames of left context

    def decode(self, codes: torch.Tensor):
        """Codes (frames, G) to a 24 kHz waveform (numpy float32) and its sample rate, as the official
        ``speech_tokenizer.decode`` computes it (qwen3/fast.py:307-341). With graphs the codes are cut as the
        official chunked decode cuts them (300 frames with 25 frames of left context), each segment zero-padded to a
        bucket length and decoded by that bucket's graph, then trimmed: the decoder is causal, so padding on the
        right leaves the earlier samples unchanged."""
        tok = self.model.speech_tokenizer
        if not self.graphs:
            wavs, sr = tok.decode([{"audio_codes": codes}])
            return wavs[0], sr
        up = int(tok.model.decoder.total_upsample)
        c = torch.clamp(codes, min=0).t().unsqueeze(0)  # (1, G, frames)
        F = int(c.shape[-1])
        pieces = []
        for start in range(0, F, self.DEC_CHUNK):
            end = min(start + self.DEC_CHUNK, F)
            ctx = self.DEC_CONTEXT if start > self.DEC_CONTEXT else start
            pieces.append(self._decode_segment(c[..., start - ctx:end])[..., ctx * up:])
        wav = torch.cat(pieces, dim=-1).reshape(-1)[: F * int(tok.model.decode_upsample_rate)]
        return wav.to(torch.float32).cpu().numpy(), int(tok.model.get_output_sample_rate())

    def _decode_segment(self, seg: torch.Tensor) -> torch.Tensor:
        n = int(seg.shape[-1])
        B = next((b for b in self.DEC_BUCKETS if b >= n), None)
        if B is None:
            raise ValueError(f"a decode segment of {n} frames exceeds the largest bucket {self.DEC_BUCKETS[-1]}")
        if B not in self._dec:
            self._dec[B] = self._capture_decode(B)
        g, buf, out = self._dec[B]
        buf.zero_()
        buf[..., :n].copy_(seg)
        g.replay()
        up = int(self.model.speech_tokenizer.model.decoder.total_upsample)
        return out[..., : n * up].clone()

    def _capture_decode(self, B: int):
        """Records the decoder over a (1, G, B) code buffer: two warm-up runs on a side stream, then the capture."""
        t0 = time.perf_counter()
        dec = self.model.speech_tokenizer.model.decoder
        buf = torch.zeros((1, self.G, B), dtype=torch.long, device=self.device)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(2):
                dec(buf)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=self._pool), torch.inference_mode():
            out = dec(buf)
        torch.cuda.synchronize()
        self.stats["decode_capture_sec"] = self.stats.get("decode_capture_sec", 0.0) + time.perf_counter() - t0
        return g, buf, out

    def warm_decode(self, buckets=None) -> float:
        """Records the decode graphs of the given buckets (all of them by default); returns the seconds spent."""
        t0 = time.perf_counter()
        if self.graphs:
            for B in buckets or self.DEC_BUCKETS:
                if B not in self._dec:
                    self._dec[B] = self._capture_decode(B)
        return time.perf_counter() - t0

    # --- one sentence ---------------------------------------------------------------------------------------
    def _sync(self) -> None:
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)

    @torch.no_grad()
    def synth(self, text: str, speaker: str, language: str, max_frames: int | None = None, **gen):
        """Prompt, frames, decode for one sentence (qwen3/fast.py:375-388). Returns (waveform, sample rate, codes);
        ``stats`` gets the seconds of each phase (prompt, generate, decode)."""
        t0 = time.perf_counter()
        self.stats = {}
        kw = self.prompt(text, speaker, language, **gen)
        self._sync()
        t1 = time.perf_counter()
        codes = self.generate_codes(kw, max_frames=max_frames)
        self._sync()
        t2 = time.perf_counter()
        wav, sr = self.decode(codes)
        self._sync()
        t3 = time.perf_counter()
        self.stats.update({"prompt": t1 - t0, "generate": t2 - t1, "decode": t3 - t2})
        return wav, sr, codes

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
