"""The talker decode engine on hand-written gfx950 kernels, behind the reference's ``Qwen3Kernels`` surface.

Mirrors qwen3/kernels.py: ``_Lin`` (425-447) packs one [N, K] matrix, ``_Stack`` (450-480) packs a decoder
stack, ``Qwen3Kernels`` (483-754) composes the frame. One decoder layer is five launches on the caller's stream:

  1. sk_rms_gemv(qkv)          RMSNorm fused into the q/k/v projection
  2. sk_attn                   q/k RMSNorm, RoPE, KV append, split-K GQA attention with log-sum-exp merge
  3. sk_gemv(o, accumulate)    output projection added into the fp32 residual
  4. sk_rms_gemv(gu, swiglu)   RMSNorm fused into gate/up (rows interleaved), silu(gate) * up
  5. sk_gemv(down, accumulate) down projection added into the residual

The frame (talker half of qwen3/kernels.py:676-685) is embed(id0) -> 28 layers -> sk_rmsnorm -> codec head ->
sk_sample, and is recorded once as a HIP graph. Weight formats: ``i8row`` (int8 + bf16 scale per output row,
the primary format), ``i8g32`` (the reference's int8 + fp16 per-32 scale), ``bf16`` and ``f32``.
"""

from __future__ import annotations

import ctypes
import time

import torch

from . import _lib
from .fast import Qwen3Fast, Sampling, _sample
from .sampler import FusedSampler

HD = 128


def _engine_kv_cache(config, max_len: int, kc: torch.Tensor, vc: torch.Tensor):
    """The engine's talker cache as a transformers ``StaticCache`` whose layers' key and value tensors are views of
    ``kc[i]`` / ``vc[i]`` ([nkv, max_len, 128] -> [1, nkv, max_len, 128], the same memory layout), so the talker's
    Hugging Face modules write a prompt's keys and values straight into the cache the kernels read (the reference
    shares the StaticCache tensors the same way, qwen3/kernels.py:695-703). transformers 5 static layers keep their own
    write position instead of reading ``cache_position``; ``seek(pos)`` sets it (every layer, on the device, so it
    can be recorded in a graph). A model computing in another precision than the cache attends over this call's rows
    in its own precision and over earlier rows as stored."""
    from transformers import StaticCache
    from transformers.cache_utils import StaticLayer

    class _ViewLayer(StaticLayer):
        def __init__(self, keys: torch.Tensor, values: torch.Tensor):
            super().__init__(max_cache_len=int(keys.shape[1]))
            self.keys, self.values = keys.unsqueeze(0), values.unsqueeze(0)
            self.dtype, self.device = keys.dtype, keys.device
            self.batch_size, self.num_heads = 1, int(keys.shape[0])
            self.k_head_dim = self.v_head_dim = int(keys.shape[-1])
            self.cumulative_length = torch.zeros((), dtype=torch.long, device=keys.device)
            self.is_initialized = True

        def update(self, key_states, value_states, *args, **kwargs):
            idx = torch.arange(int(key_states.shape[-2]), device=self.device) + self.cumulative_length
            self.cumulative_length.add_(int(key_states.shape[-2]))
            self.keys.index_copy_(2, idx, key_states.to(self.dtype))
            self.values.index_copy_(2, idx, value_states.to(self.dtype))
            if key_states.dtype == self.dtype:
                return self.keys, self.values
            k, v = self.keys.to(key_states.dtype), self.values.to(value_states.dtype)
            k.index_copy_(2, idx, key_states)
            v.index_copy_(2, idx, value_states)
            return k, v

        def reset(self) -> None:
            self.cumulative_length.zero_()

    class _EngineCache(StaticCache):
        def seek(self, pos: int = 0) -> None:
            for layer in self.layers:
                layer.cumulative_length.fill_(int(pos))

    cache = _EngineCache(config=config, max_cache_len=max_len)
    if len(cache.layers) != kc.shape[0]:
        raise ValueError(f"the talker config has {len(cache.layers)} layers, the engine's cache {kc.shape[0]}")
    cache.layers = [_ViewLayer(kc[i], vc[i]) for i in range(kc.shape[0])]
    return cache


class _Lin:
    """One matrix [N, K] in the kernels' format. ``wd``: ``i8row`` int8 + bf16 scale per row
    (s = bf16(max(max|w|/127, 1e-12)), q = clamp(round_half_even(w/s), +-127)); ``i8g32`` int8 + fp16 scale per
    32 K elements (qwen3/kernels.py:438-442); ``bf16``; ``f32``. ``pol`` 1 streams the weights past the caches
    (read once per frame), 0 keeps them cacheable; ``split`` is kept for interface parity (always 1)."""

    def __init__(self, w: torch.Tensor, wd: str):
        dev = w.device
        # quantise on the CPU: its fp32 division is correctly rounded, so the int8 values are reproducible
        # bit for bit on any host (a GPU division can land on the other side of a .5 tie)
        w = w.detach().to("cpu").contiguous()
        self.N, self.K = w.shape
        self.pol = 0
        self.split = 1
        self.wd = wd
        if self.K % 512 != 0:
            raise ValueError(f"K={self.K} must be a multiple of 512")
        if wd == "bf16":
            self.w, self.s = w.to(torch.bfloat16).contiguous(), None
        elif wd == "f32":
            self.w, self.s = w.float().contiguous(), None
        elif wd == "i8row":
            wf = w.float()
            sc = (wf.abs().amax(1) / 127).clamp_min(1e-12).to(torch.bfloat16)
            q = torch.round(wf / sc.float()[:, None])
            q = torch.nan_to_num(q, nan=0.0).clamp(-127, 127).to(torch.int8)
            self.w, self.s = q.contiguous(), sc.view(torch.int16).contiguous()
        elif wd == "i8g32":
            g = w.float().view(self.N, self.K // 32, 32)
            sc = (g.abs().amax(2) / 127).clamp_min(1e-12).half()
            q = torch.round(g / sc.float()[..., None])
            q = torch.nan_to_num(q, nan=0.0, posinf=127.0, neginf=-127.0).clamp(-127, 127).to(torch.int8)
            self.w, self.s = q.view(self.N, self.K).contiguous(), sc.view(torch.int16).contiguous()
        else:
            raise ValueError(wd)
        self.w = self.w.to(dev)
        self.s = None if self.s is None else self.s.to(dev)

    @property
    def wd_code(self) -> int:
        return _lib.WD[self.wd]

    def bytes(self) -> int:
        return self.w.numel() * self.w.element_size() + (0 if self.s is None else self.s.numel() * 2)

    def dequant(self) -> torch.Tensor:
        """fp32 [N, K] weights the kernels effectively multiply with (for checks)."""
        if self.wd in ("bf16", "f32"):
            return self.w.float()
        if self.wd == "i8row":
            return self.w.float() * self.s.view(torch.bfloat16).float()[:, None]
        s = self.s.view(torch.float16).float()
        return (self.w.float().view(self.N, self.K // 32, 32) * s[..., None]).view(self.N, self.K)


class _Stack:
    """Decoder layers in kernel form (qwen3/kernels.py:450-480): q/k/v rows concatenated into ``qkv``, gate/up
    rows interleaved (row 2n gate n, row 2n+1 up n) into ``gu``, norm weights fp32, and the RoPE table
    [max_len][cos 64 | sin 64] from ``pos * inv_freq`` in fp32."""

    def __init__(self, model, wd: str, max_len: int):
        cfg = model.config
        self.H, self.I = int(cfg.hidden_size), int(cfg.intermediate_size)
        self.nq, self.nkv = int(cfg.num_attention_heads), int(cfg.num_key_value_heads)
        if int(cfg.head_dim) != HD or self.nq != 2 * self.nkv:
            raise ValueError("only head_dim 128 with two q heads per kv head is supported")
        self.eps = float(cfg.rms_norm_eps)
        self.layers = []
        for layer in model.layers:
            a, m = layer.self_attn, layer.mlp
            gu = torch.stack([m.gate_proj.weight, m.up_proj.weight], dim=1).reshape(2 * self.I, self.H)
            self.layers.append({
                "in_norm": layer.input_layernorm.weight.float().contiguous(),
                "qkv": _Lin(torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], dim=0), wd),
                "qn": a.q_norm.weight.float().contiguous(), "kn": a.k_norm.weight.float().contiguous(),
                "o": _Lin(a.o_proj.weight, wd),
                "post_norm": layer.post_attention_layernorm.weight.float().contiguous(),
                "gu": _Lin(gu, wd), "down": _Lin(m.down_proj.weight, wd),
            })
            if getattr(a.q_proj, "bias", None) is not None or getattr(a.o_proj, "bias", None) is not None:
                raise ValueError("attention biases are not supported")
        self.norm = model.norm.weight.float().contiguous()
        inv = model.rotary_emb.inv_freq.float()
        if inv.numel() != HD // 2 or float(model.rotary_emb.attention_scaling) != 1.0:
            raise ValueError("only default 1-D RoPE (64 frequencies, scaling 1) is supported")
        f = torch.arange(max_len, device=inv.device, dtype=torch.float32)[:, None] * inv[None, :]
        self.rope = torch.cat([f.cos(), f.sin()], dim=1).contiguous()
        self.max_len = max_len

    def bytes(self) -> int:
        return sum(L[k].bytes() for L in self.layers for k in ("qkv", "o", "gu", "down"))


def _keep_policies(layers: list, l2_keep_mb: float | None) -> int:
    """Cache policy of the code predictor's matrices (qwen3/kernels.py:525-542): walking the layers in order, a
    matrix that fits the remaining budget of ``l2_keep_mb`` MiB stays cacheable (``pol`` 0) and uses up its
    bytes, one that does not is streamed (``pol`` 1). ``None`` is an unbounded budget. Returns the kept bytes."""
    budget = float("inf") if l2_keep_mb is None else float(l2_keep_mb) * 2**20
    kept = 0
    for Ly in layers:
        for m in ("qkv", "o", "gu", "down"):
            b = Ly[m].bytes()
            Ly[m].pol = 0 if b <= budget else 1
            if b <= budget:
                budget -= b
                kept += b
    return kept


def _sptr(lin: "_Lin") -> int:
    """Device address of a matrix's scales, 0 for the formats without (bf16, f32)."""
    return 0 if lin.s is None else lin.s.data_ptr()


def place_cells(ws: torch.Tensor, attempts: int = 3) -> int:
    """Measures where a zeroed frame-kernel workspace's exchange cells go (``sk_frames_place``: each XCD's copy on
    the page nearest it) on the current stream, and returns how many of the cell region's four quarters got a
    measured placement. A quarter whose measurement was not consistent keeps the fixed placement (same results,
    slower exchanges); the measurement is repeated for it up to ``attempts`` times in all (each waits for the
    stream). Called after every zeroing of the workspace; the launches read the result from the workspace."""
    L = _lib.load()
    placed = 0
    for _ in range(max(1, attempts)):
        _lib.check(L.sk_frames_place(ws.data_ptr(), ws.numel(), _lib.stream()), "sk_frames_place")
        words = ws[48:64].view(torch.int32).tolist()
        placed = sum(1 for w in words if w < 0)  # bit 31: a measured quarter
        if placed == len(words):
            break
    return placed


def _layer_descs(P: _Stack, kc: list, vc: list, device) -> torch.Tensor:
    """Device array of ``sk_layer_desc`` for the layers of ``P`` with caches ``kc[i]`` / ``vc[i]``."""
    arr = (_lib.SkLayerDesc * len(P.layers))()
    for i, Ly in enumerate(P.layers):
        arr[i] = _lib.SkLayerDesc(Ly["qkv"].w.data_ptr(), _sptr(Ly["qkv"]), Ly["o"].w.data_ptr(),
                                  _sptr(Ly["o"]), Ly["gu"].w.data_ptr(), _sptr(Ly["gu"]),
                                  Ly["down"].w.data_ptr(), _sptr(Ly["down"]), Ly["in_norm"].data_ptr(),
                                  Ly["post_norm"].data_ptr(), Ly["qn"].data_ptr(), Ly["kn"].data_ptr(),
                                  kc[i].data_ptr(), vc[i].data_ptr())
    return torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8).to(device)


class CodePredictor:
    """The code predictor of one frame on the persistent kernel in its code-predictor mode (``sk_cp_frame``).

    Weights as the reference reads them (qwen3/kernels.py:516-523): ``cp.model`` (its decoder stack, packed by
    ``_Stack`` with a cache of ``n_positions``), ``cp.lm_head`` (head g - 1 produces code g) and
    ``cp.get_input_embeddings()`` (table g - 2 embeds code g - 1 at position g). The loop is the reference's
    (qwen3/kernels.py:666-675 with ``_cp_first`` 641-655): position 0 takes the talker's last hidden state,
    position 1 the talker embedding row of code 0, position g >= 2 the embedding of code g - 1; each position
    g >= 1 ends in the final RMSNorm, head g - 1 and a pick: greedy, or after ``set_sampling`` the fused
    sampler's draw (temperature, top_k, Philox seed and counter in device memory; one draw per position g >= 1).
    A code predictor narrower than the talker (``cp.small_to_mtp_projection`` not the identity, the 1.7B Qwen3-TTS)
    projects every position's input, with the projection's bias, before its layers (``_cp_input``,
    qwen3/kernels.py:629-637): ``x0`` and the tables are then the talker's width."""

    def __init__(self, cp, temb: torch.Tensor, n_positions: int = 16, wd: str = "i8row", device=None,
                 x0: torch.Tensor | None = None, id0: torch.Tensor | None = None, codes: torch.Tensor | None = None,
                 keep_layers: bool = True, pair: bool | None = None):
        """``x0`` (fp32 [hidden]), ``id0`` (int64, one element) and ``codes`` (int64 [n_positions]) may be a caller's
        own contiguous device buffers: the kernel then reads and writes them in place (no copies per frame).
        ``keep_layers`` loads the layer weights through the caches (read once per position, they stay in L2 and
        the Infinity Cache across the frame) instead of streaming them like the heads (``sk_cp_desc.keep_layers``).
        ``pair`` runs positions 0 and 1 as one pass with two rows per stage (the reference's cp_pair,
        qwen3/kernels.py:600-617; ``sk_cp_desc.pair``); by default on, and off for a projected code predictor,
        which the kernel runs unpaired."""
        if wd not in ("i8row", "i8g32", "bf16"):
            raise ValueError("the code-predictor kernel reads i8row, i8g32 or bf16 weights")
        proj = getattr(cp, "small_to_mtp_projection", None)
        projected = proj is not None and not isinstance(proj, torch.nn.Identity)
        if pair is None:
            pair = not projected
        if projected and pair:
            raise NotImplementedError("a projected code predictor runs unpaired on sk_cp_frame (pair=False)")
        L = _lib.load()
        self.device = torch.device(device) if device is not None else temb.device
        self.n = int(n_positions)
        with torch.no_grad():
            self.C = _Stack(cp.model, wd, self.n)
            self.heads = [_Lin(h.weight, wd) for h in cp.lm_head][: self.n - 1]
            self.cemb = [e.weight.to(torch.bfloat16).contiguous() for e in cp.get_input_embeddings()][: self.n - 2]
            self.temb = temb.to(torch.bfloat16).contiguous()
            self.proj = None
            if projected:
                bias = getattr(proj, "bias", None)
                self.proj = (_Lin(proj.weight, wd), None if bias is None else bias.float().contiguous().to(self.device))
        if len(self.heads) != self.n - 1 or len(self.cemb) != self.n - 2:
            raise ValueError(f"{self.n} positions need {self.n - 1} heads and {self.n - 2} code tables")
        P = self.C
        self.V = self.heads[0].N
        dev = self.device
        self.kc = torch.zeros((len(P.layers), P.nkv, self.n, HD), dtype=torch.bfloat16, device=dev)
        self.vc = torch.zeros_like(self.kc)
        def bind(t, n, dtype):
            if t is None:
                return torch.zeros(n, dtype=dtype, device=dev)
            if t.numel() != n or t.dtype != dtype or not t.is_contiguous() or t.device != dev:
                raise ValueError(f"a bound buffer must be a contiguous {dtype} tensor of {n} elements on {dev}")
            return t.view(n)

        self.in_width = self.proj[0].K if self.proj is not None else P.H  # the width of x0 and of the tables' rows
        if self.temb.shape[1] != self.in_width or any(t.shape[1] != self.in_width for t in self.cemb):
            raise ValueError(f"the input tables must be {self.in_width} wide")
        self.x0 = bind(x0, self.in_width, torch.float32)
        self.id0 = bind(id0, 1, torch.int64)
        self.codes = bind(codes, self.n, torch.int64)
        self.logits = torch.zeros(self.V, dtype=torch.float32, device=dev)
        self.layer_out: torch.Tensor | None = None
        tabs = [0, self.temb.data_ptr()] + [t.data_ptr() for t in self.cemb]
        hw = [0] + [h.w.data_ptr() for h in self.heads]
        hs = [0] + [_sptr(h) for h in self.heads]
        self._ptrs = torch.tensor([tabs, hw, hs], dtype=torch.int64, device=dev)
        self._layer_desc = _layer_descs(P, list(self.kc.unbind(0)), list(self.vc.unbind(0)), dev)
        self.ws = torch.zeros(int(L.sk_cp_workspace_size(P.H, P.I, int(bool(pair)))), dtype=torch.uint8, device=dev)
        place_cells(self.ws)
        self._desc = _lib.SkCpDesc(
            n_layers=len(P.layers), hidden=P.H, inter=P.I, nq=P.nq, nkv=P.nkv, vocab=self.V, n_positions=self.n,
            wd=_lib.WD[wd], ct=_lib.CT["bf16"], eps=P.eps, layers=self._layer_desc.data_ptr(), norm=P.norm.data_ptr(),
            rope=P.rope.data_ptr(), x0=self.x0.data_ptr(), id0=self.id0.data_ptr(), emb0_rows=self.temb.shape[0],
            emb=self._ptrs[0].data_ptr(), head_w=self._ptrs[1].data_ptr(), head_s=self._ptrs[2].data_ptr(),
            codes=self.codes.data_ptr(), logits=self.logits.data_ptr(), layer_out=None,
            workspace=self.ws.data_ptr(), workspace_bytes=self.ws.numel(), keep_layers=int(bool(keep_layers)),
            pair=int(bool(pair)))
        if self.proj is not None:
            pw, pb = self.proj
            self._desc.proj_in = pw.K
            self._desc.proj_w = pw.w.data_ptr()
            self._desc.proj_s = _sptr(pw)
            self._desc.proj_b = None if pb is None else pb.data_ptr()
        self.keep_layers = bool(keep_layers)
        self.pair = bool(pair)
        self.wd = wd
        self.graph: torch.cuda.CUDAGraph | None = None

    def set_sampling(self, temperature: float, top_k: int, seed: torch.Tensor, counter: torch.Tensor) -> None:
        """Sampled sub-codes from here on: position g >= 1 draws with counter ``counter + g - 1`` under key
        ``seed`` (device int64 tensors, as the fused sampler keeps them), and ``counter`` advances by
        ``n_positions - 1`` per frame. Call before ``capture``: a graph keeps the settings it was recorded with."""
        if not temperature > 0:
            raise ValueError("temperature must be positive")
        self._desc.do_sample = 1
        self._desc.inv_temp = 1.0 / float(temperature)
        self._desc.top_k = int(top_k or 0)
        self._seed, self._counter = seed, counter  # keep the tensors alive
        self._desc.seed = seed.data_ptr()
        self._desc.counter = counter.data_ptr()

    def run(self) -> None:
        """One frame on the current stream: reads ``x0`` and ``id0``, writes ``codes`` (and ``logits`` of the
        last position)."""
        self._desc.layer_out = None if self.layer_out is None else self.layer_out.data_ptr()
        _lib.check(_lib.load().sk_cp_frame(ctypes.byref(self._desc), _lib.stream()), "sk_cp_frame")

    def __call__(self, x0: torch.Tensor, id0) -> torch.Tensor:
        self.x0.copy_(x0.reshape(-1))
        self.id0.fill_(int(id0)) if not isinstance(id0, torch.Tensor) else self.id0.copy_(id0.reshape(1))
        self.run()
        return self.codes

    def capture(self) -> None:
        """Records one frame (one launch) as a HIP graph; replays read ``x0`` / ``id0`` in place."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.run()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.run()
        torch.cuda.synchronize()
        self.graph = g

    def error(self) -> int:
        """Error word of the kernel's workspace (0 when healthy; codes as ``Qwen3Kernels.frame_error``)."""
        return int(self.ws[:4].view(torch.int32).item())

    def diag(self) -> dict:
        w = self.ws[16:32].view(torch.int32).tolist()
        return {"code": w[0], "frame": w[1], "layer": w[2], "workgroup": w[3]}

    def clear_error(self) -> None:
        """Zeroes the kernel's whole workspace (error word, launch census, epoch base and exchange cells), so the
        next launch starts clean after a failed one, and places its cells again (``place_cells``, which waits for
        the current stream); not to be called while a launch of this code predictor may be in flight on another
        stream."""
        self.ws.zero_()
        place_cells(self.ws)

    def weight_bytes(self) -> int:
        return self.C.bytes() + sum(h.bytes() for h in self.heads) + (self.proj[0].bytes() if self.proj else 0)


class Qwen3Kernels(Qwen3Fast):
    """The talker frame on the sokutou_amd kernels (qwen3/kernels.py:483-754 surface).

    Constructor arguments as the reference; ``wd`` adds ``i8row``. ``l2_keep_mb`` is the reference's cache budget
    for the code predictor's layers (qwen3/kernels.py:525-542): matrices within it, in layer order, are loaded
    cacheable (policy 0), the rest and every talker and head weight are streamed (policy 1); unset, it covers all
    of them (their 79 MB fit MI355X's 256 MB Infinity Cache). The one-launch code-predictor kernel applies one
    policy to all its layers: cacheable only when the budget covers every layer. ``cp_pair`` (default on, as the
    reference) runs the code predictor's positions 0 and 1 as one pass on the one-launch kernel; the per-kernel
    path runs them one after the other. ``suppress_tail`` (default 1024, as the reference) sets how many trailing ids the
    processor suppresses; 0 disables suppression.
    """

    def __init__(self, tts, sampling: Sampling | None = None, max_cache: int = 1024, wd: str = "bf16",
                 graphs: bool = True, sampler: str = "fused", l2_keep_mb: float | None = None,
                 cp_pair: bool | None = None, suppress_tail: int = 1024, frame_kernel: bool | None = None):
        super().__init__(tts, sampling, max_cache=max_cache, compile=False, graphs=graphs, suppress_tail=suppress_tail)
        if sampler not in ("fused", "torch"):
            raise ValueError(sampler)
        if wd not in _lib.WD:
            raise ValueError(wd)
        L = _lib.load()
        if self.device.type != "cuda":
            raise RuntimeError("Qwen3Kernels runs on a HIP device")
        with torch.cuda.device(self.device):
            _lib.check(L.sk_device_check(), "sk_device_check")
        t0 = time.perf_counter()
        self.wd = wd
        self.ct = "f32" if wd == "f32" else "bf16"
        cdt = torch.float32 if self.ct == "f32" else torch.bfloat16
        self.cp_pair = bool(cp_pair) if cp_pair is not None else True
        self._l2_keep_arg = l2_keep_mb
        self.l2_keep_mb = l2_keep_mb if l2_keep_mb is not None else 0.0
        dev = self.device
        with torch.no_grad():
            self.T = _Stack(self.talker.model, wd, max_cache)
            self.codec_head = _Lin(self.talker.codec_head.weight, wd)
            self.temb = self.talker.get_input_embeddings().weight.to(cdt).contiguous()
        for Ly in self.T.layers:
            for m in ("qkv", "o", "gu", "down"):
                Ly[m].pol = 1
        self.codec_head.pol = 1
        self.l2_kept_bytes = 0
        self.kernel_compile_sec = time.perf_counter() - t0
        self.sampler = sampler
        self.fs = FusedSampler(dev) if sampler == "fused" else None
        P = self.T
        f32 = dict(dtype=torch.float32, device=dev)
        self.ph32 = torch.zeros(P.H, **f32)
        self.ht = torch.zeros(P.H, **f32)
        self.qkv_t = torch.zeros((P.nq + 2 * P.nkv) * HD, **f32)
        self.att_t = torch.zeros(P.nq * HD, **f32)
        self.act_t = torch.zeros(P.I, **f32)
        self.logit_t = torch.zeros((1, self.V), **f32)
        # talker KV cache [layer][kv head][position][128]
        self.kc = torch.zeros((len(P.layers), P.nkv, max_cache, HD), dtype=cdt, device=dev)
        self.vc = torch.zeros_like(self.kc)
        self.tk = list(self.kc.unbind(0))
        self.tv = list(self.vc.unbind(0))
        # the same cache for the talker's Hugging Face modules (the prompt prefill), when they are runnable
        hf_cfg = getattr(getattr(self.talker, "model", None), "config", None)
        self.tcache = (_engine_kv_cache(hf_cfg, max_cache, self.kc, self.vc)
                       if hasattr(hf_cfg, "get_text_config") and callable(self.talker.model) else None)
        nbytes = int(L.sk_attn_workspace_size(P.nq, P.nkv, max_cache))
        self.attn_ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        self.trace: list[torch.Tensor] | None = None
        if self.cp is not None:
            self._setup_code_predictor(wd, cdt)
        # whole frames in one persistent launch (0.6B / 1.7B talker shapes; greedy or the fused sampler's draw)
        supported = (self.frame_kernel_supported() and sampler == "fused"
                     and (self.cp is None or self.cpk is not None))
        if frame_kernel and not supported:
            raise ValueError("frame_kernel=True needs the fused sampler, i8row, i8g32 or bf16 weights, "
                             "16 q / 8 kv heads, vocab 3072, "
                             "hidden 1024 or 2048, a cache of at most 1024 (0.6B) / 2048 (1.7B) positions and, with a "
                             "code predictor, its one-launch kernel (the 1024-wide code predictor, unprojected or "
                             "projected from 2048)")
        self.frame_kernel = supported if frame_kernel is None else bool(frame_kernel)
        if self.frame_kernel:
            self._setup_frame_kernel()

    # --- the code predictor -----------------------------------------------------------------------------------
    def _setup_code_predictor(self, wd: str, cdt) -> None:
        """The code predictor's stack, heads, code tables and optional projection (qwen3/kernels.py:514-523), its
        cache [layers, nkv, G, 128] and buffers. Sub-codes of the 1024-wide code predictor (the 0.6B Qwen3-TTS's,
        and the 1.7B's behind its projection from the talker's 2048-wide rows) run on the one-launch kernel
        (CodePredictor); anything else runs position by position on the per-op kernels, as the reference does
        (qwen3/kernels.py:629-675)."""
        cp, dev = self.cp, self.device
        with torch.no_grad():
            self.C = _Stack(cp.model, wd, self.G)
            self.cp_heads = [_Lin(h.weight, wd) for h in cp.lm_head][: self.G - 1]
            self.cemb = [e.weight.to(cdt).contiguous() for e in cp.get_input_embeddings()]
            proj = getattr(cp, "small_to_mtp_projection", None)
            self.proj = None
            if proj is not None and not isinstance(proj, torch.nn.Identity):
                bias = getattr(proj, "bias", None)
                self.proj = (_Lin(proj.weight, wd), None if bias is None else bias.float().contiguous())
        if len(self.cp_heads) != self.G - 1 or len(self.cemb) < self.G - 1:
            raise ValueError(f"{self.G} code groups need {self.G - 1} heads and {self.G - 1} code tables")
        for h in self.cp_heads:
            h.pol = 1
        self.l2_kept_bytes = _keep_policies(self.C.layers, self._l2_keep_arg)
        if self._l2_keep_arg is None:
            self.l2_keep_mb = self.l2_kept_bytes / 2**20
        # talker input tables: code 0 from the talker's table, code g >= 1 from code table g - 1
        self.tabs = torch.tensor([self.temb.data_ptr()] + [e.data_ptr() for e in self.cemb[: self.G - 1]],
                                 dtype=torch.int64, device=dev)
        P = self.C
        f32 = dict(dtype=torch.float32, device=dev)
        self.pad16 = torch.zeros(self.T.H, dtype=cdt, device=dev)  # tts_pad_embed, added to every talker input
        self.hc = torch.zeros(P.H, **f32)
        self.e = torch.zeros(self.T.H, **f32)
        self.qkv_c = torch.zeros((P.nq + 2 * P.nkv) * HD, **f32)
        self.att_c = torch.zeros(P.nq * HD, **f32)
        self.act_c = torch.zeros(P.I, **f32)
        self.logit_c = torch.zeros((1, self.cp_heads[0].N), **f32)
        self.ck = torch.zeros((len(P.layers), P.nkv, self.G, HD), dtype=cdt, device=dev)
        self.cv = torch.zeros_like(self.ck)
        self.cpk: CodePredictor | None = None
        # the one-launch kernel takes the 1024-wide code predictor, unprojected or behind a projection from the 1.7B
        # talker's 2048-wide rows (then unpaired)
        fast = ((not self.s.sub_do_sample or self.fs is not None)
                and (self.proj is None or self.proj[0].K == 2048)
                and wd in ("i8row", "i8g32", "bf16")
                and self.ct == "bf16" and (P.H, P.I, P.nq, P.nkv, self.cp_heads[0].N) == (1024, 3072, 16, 8, 2048)
                and 2 <= self.G <= 64)
        if fast:
            # bound to the frame state: reads ph32 and code 0, writes all G codes, with no copy per frame
            keep = all(Ly[m].pol == 0 for Ly in P.layers for m in ("qkv", "o", "gu", "down"))
            self.cpk = CodePredictor(cp, self.temb, n_positions=self.G, wd=wd, device=dev, x0=self.ph32, id0=self.id0,
                                     codes=self.codes, keep_layers=keep, pair=self.cp_pair and self.proj is None)
            if self.s.sub_do_sample:  # the fused sampler's draws, in the same order as position by position
                self.cpk.set_sampling(self.s.sub_temperature, self.s.sub_top_k, self.fs.seed, self.fs.counter)

    def _cp_input(self, x) -> None:
        """Code-predictor input from a talker-width fp32 vector: the projection (with its bias) or a copy
        (qwen3/kernels.py:629-637)."""
        if self.proj is None:
            self.hc.copy_(x)
        else:
            self._gemv(x, self.proj[0], self.proj[1], self.hc, False)

    def _cp_frame(self) -> None:
        """Sub-codes 1..G-1 of the frame into ``codes`` from ph32 (the talker's last hidden state after its final
        norm) and code 0 (qwen3/kernels.py:666-675 with _cp_first 641-655): position 0 takes ph32, position 1 the
        talker embedding of code 0, position g >= 2 code table g - 2 at code g - 1; position g >= 1 ends in the final
        norm, head g - 1 and a pick with the sub-code settings (no processor)."""
        s, codes = self.s, self.codes
        if self.cpk is not None:  # reads ph32 and id0, writes codes[0, :G] (code 0 passes through)
            self.cpk.run()
            return
        codes[:, :1].copy_(self.id0)
        P = self.C
        cptr = codes.data_ptr()
        for g in range(self.G):
            if g == 0:
                self._cp_input(self.ph32)
            else:
                self._embed(self.temb if g == 1 else self.cemb[g - 2], self.id0 if g == 1 else cptr + 8 * (g - 1),
                            self.e)
                self._cp_input(self.e)
            self._layers(P, self.hc, self.qkv_c, self.att_c, self.act_c, list(self.ck.unbind(0)),
                         list(self.cv.unbind(0)), None, g)
            if g == 0:
                continue
            self._rms_gemv(self.hc, P.norm, P.eps, self.cp_heads[g - 1], self.logit_c, False)
            if self.fs is not None:
                self.fs(self.logit_c.view(-1), cptr + 8 * g, s.sub_do_sample, s.sub_temperature, s.sub_top_k)
            else:
                codes[:, g:g + 1].copy_(_sample(self.logit_c, s.sub_do_sample, s.sub_temperature, s.sub_top_k))

    def _state(self):
        base = super()._state()
        return base + (self.ph32,) if self.cp is not None else base

    # --- the persistent frame kernel ------------------------------------------------------------------------
    def frame_kernel_supported(self) -> bool:
        """The persistent kernel covers the 0.6B and 1.7B talker shapes with i8row weights, the reference's i8g32
        or bf16 weights (the reference's default format)."""
        P = self.T
        shapes = {(1024, 3072): 1024, (2048, 6144): 2048}
        wd_ok = self.wd in ("i8row", "i8g32", "bf16")
        return (wd_ok and self.ct == "bf16" and P.nq == 16 and P.nkv == 8 and self.V == 3072
                and (P.H, P.I) in shapes and self.max_cache <= shapes[(P.H, P.I)])

    def _setup_frame_kernel(self) -> None:
        P = self.T
        L = _lib.load()
        self._layer_desc = _layer_descs(P, self.tk, self.tv, self.device)
        self.frame_ws = torch.zeros(int(L.sk_talker_workspace_size(P.H, P.I)), dtype=torch.uint8, device=self.device)
        place_cells(self.frame_ws)
        self.frame_ids = torch.zeros(4096, dtype=torch.int64, device=self.device)
        self.layer_out: torch.Tensor | None = None
        s = self.s
        proc = s.repetition_penalty != 1.0 or self.suppress_tail != 0 or s.min_new_tokens > 0
        self._desc = _lib.SkTalkerDesc(
            n_layers=len(P.layers), hidden=P.H, inter=P.I, nq=P.nq, nkv=P.nkv, vocab=self.V, max_len=P.max_len,
            wd=_lib.WD[self.wd], ct=_lib.CT[self.ct], eps=P.eps, layers=self._layer_desc.data_ptr(),
            norm=P.norm.data_ptr(), head_w=self.codec_head.w.data_ptr(), head_s=_sptr(self.codec_head),
            emb=self.temb.data_ptr(), rope=P.rope.data_ptr(), id0=self.id0.data_ptr(), pos=self.pos.data_ptr(),
            next_id0=self.next_id0.data_ptr(), out=self.frame_ids.data_ptr(), seen=self.seen.data_ptr(),
            ngen=self.ngen.data_ptr(), suppress=self.suppress.data_ptr() if self.suppress_tail else None,
            rep_pen=s.repetition_penalty, min_new=s.min_new_tokens, eos=self.eos, talker_processor=int(proc),
            logits=self.logit_t.data_ptr(), layer_out=None, workspace=self.frame_ws.data_ptr(),
            workspace_bytes=self.frame_ws.numel())
        if s.do_sample:  # the fused sampler's draw: one counter step per frame, seed and counter shared with it
            self._desc.do_sample = 1
            self._desc.inv_temp = 1.0 / s.temperature
            self._desc.top_k = int(s.top_k or 0)
            self._desc.seed = self.fs.seed.data_ptr()
            self._desc.counter = self.fs.counter.data_ptr()
        if self.cp is not None:
            # one frame per launch, fed by talker_in of the frame's codes; the final norm's output feeds the next
            # frame's code predictor
            self._desc.in_tabs = self.tabs.data_ptr()
            self._desc.in_codes = self.codes.data_ptr()
            self._desc.in_pad = self.pad16.data_ptr()
            self._desc.in_groups = self.G
            self._desc.in_rows = min(int(e.shape[0]) for e in self.cemb[: self.G - 1])
            self._desc.final_out = self.ph32.data_ptr()

    def run_frames(self, n: int) -> None:
        """``n`` frames in one launch of sk_talker_frames; the chosen ids land in ``frame_ids[:n]``."""
        if n > self.frame_ids.numel():
            raise ValueError("at most 4096 frames per launch")
        if self.cp is not None and n != 1:
            raise ValueError("with a code predictor each launch runs one talker frame")
        self._desc.layer_out = None if self.layer_out is None else self.layer_out.data_ptr()
        _lib.check(_lib.load().sk_talker_frames(ctypes.byref(self._desc), int(n), _lib.stream()), "sk_talker_frames")

    def frame_error(self) -> int:
        """Error word of the frame kernel's workspace (0 when healthy; reads device memory, so it synchronises).
        Codes: 2 placement, 5 position/token out of range, 10 the poll of a projected code predictor's input
        timed out, 11..18 a poll of stage S1, S2, S3, S4, S5, S6, head, pick timed out, 19 the maxima of a sampled
        pick, 20 its values timed out (``frame_diag`` tells the frame, layer and workgroup)."""
        return int(self.frame_ws[:4].view(torch.int32).item())

    def frame_diag(self) -> dict:
        w = self.frame_ws[16:32].view(torch.int32).tolist()
        return {"code": w[0], "frame": w[1], "layer": w[2], "workgroup": w[3]}

    def clear_frame_error(self) -> None:
        """Clears every device error word of the engine so frames can run again after a failure: the frame kernel's
        and the one-launch code predictor's whole workspaces (error word, launch census, epoch base and exchange cells
        all restart from zero, so no stale cell can match a new epoch, and the cells are placed again, which waits for
        the current stream) and the attention workspace's error word."""
        if self.frame_kernel:
            self.frame_ws.zero_()
            place_cells(self.frame_ws)
        if self.cp is not None and self.cpk is not None:
            self.cpk.clear_error()
        self.attn_ws[:4].zero_()

    def _check_errors(self) -> None:
        """Reads the device error words of the kernels this engine runs (frame kernel, one-launch code predictor,
        per-op attention) and raises RuntimeError naming the first one set; clear_frame_error() resets them."""
        words = []
        if self.frame_kernel:
            words.append(("sk_talker_frames", self.frame_ws, self.frame_diag))
        if self.cp is not None and self.cpk is not None:
            words.append(("sk_cp_frame", self.cpk.ws, self.cpk.diag))
        words.append(("sk_attn", self.attn_ws, None))
        for name, ws, diag in words:
            code = int(ws[:4].view(torch.int32).item())
            if code:
                extra = f" {diag()}" if diag is not None else ""
                raise RuntimeError(f"{name} reported device error {code}{extra}; the frame state was not advanced "
                                   f"(clear_frame_error() resets the error words)")

    # --- launches -----------------------------------------------------------------------------------------
    def _rms_gemv(self, h, nw, eps, lin: _Lin, out, swiglu: bool) -> None:
        p = _lib.ptr
        _lib.call("sk_rms_gemv", p(h), p(nw), float(eps), p(lin.w), p(lin.s), p(out), lin.N, lin.K, int(swiglu),
                  lin.wd_code, lin.pol, _lib.stream())

    def _gemv(self, x, lin: _Lin, bias, out, accumulate: bool) -> None:
        p = _lib.ptr
        _lib.call("sk_gemv", p(x), p(lin.w), p(lin.s), p(bias), p(out), lin.N, lin.K, int(accumulate), lin.wd_code,
                  lin.pol, _lib.stream())

    def _attn(self, P: _Stack, L: dict, qkv, kc, vc, pos_ptr, pos_add: int, out) -> None:
        p = _lib.ptr
        _lib.call("sk_attn", p(qkv), p(L["qn"]), p(L["kn"]), float(P.eps), p(P.rope), p(kc), p(vc), p(pos_ptr),
                  int(pos_add), P.max_len, P.nq, P.nkv, p(out), p(self.attn_ws), self.attn_ws.numel(),
                  _lib.CT[self.ct], _lib.stream())

    def _embed(self, table, idx, out) -> None:
        p = _lib.ptr
        _lib.call("sk_embed", p(table), p(idx), p(out), out.numel(), _lib.CT[self.ct], _lib.stream())

    def _rmsnorm(self, h, nw, eps, out) -> None:
        p = _lib.ptr
        _lib.call("sk_rmsnorm", p(h), p(nw), float(eps), p(out), h.numel(), _lib.stream())

    def _layers(self, P: _Stack, h, qkv, att, act, kcache, vcache, pos_ptr, pos_add: int) -> None:
        """One decoder stack on the fp32 residual ``h`` (qwen3/kernels.py:619-627)."""
        for i, L in enumerate(P.layers):
            self._rms_gemv(h, L["in_norm"], P.eps, L["qkv"], qkv, False)
            self._attn(P, L, qkv, kcache[i], vcache[i], pos_ptr, pos_add, att)
            self._gemv(att, L["o"], None, h, True)
            self._rms_gemv(h, L["post_norm"], P.eps, L["gu"], act, True)
            self._gemv(act, L["down"], None, h, True)
            if self.trace is not None:
                self.trace.append(h.clone())

    # --- one frame ----------------------------------------------------------------------------------------
    def _talker(self) -> None:
        """Input -> layers -> final RMSNorm -> codec head (logits in ``logit_t``). The input is the embedding of
        code 0, or, with a code predictor, the sum of the embeddings of the frame's G codes plus the pad embedding
        (talker_in, qwen3/kernels.py:686-687)."""
        P = self.T
        if self.cp is not None:
            p = _lib.ptr
            _lib.call("sk_talker_in", p(self.tabs), p(self.codes), p(self.pad16), p(self.ht), P.H, self.G,
                      _lib.CT[self.ct], _lib.stream())
        else:
            self._embed(self.temb, self.id0, self.ht)
        self._layers(P, self.ht, self.qkv_t, self.att_t, self.act_t, self.tk, self.tv, self.pos, 0)
        self._rmsnorm(self.ht, P.norm, P.eps, self.ph32)
        self._gemv(self.ph32, self.codec_head, None, self.logit_t, False)

    def _frame(self) -> None:
        s = self.s
        if self.cp is not None:
            self._cp_frame()
        else:
            self.codes[:, :1].copy_(self.id0)
        if self.frame_kernel:
            self.run_frames(1)
            return
        self._talker()
        if self.fs is not None:
            # processor and the state update (next_id0, id0, seen, ngen, pos) happen inside the kernel
            self.fs(self.logit_t.view(-1), self.next_id0, s.do_sample, s.temperature, s.top_k,
                    talker=dict(seen=self.seen, rep_pen=s.repetition_penalty,
                                suppress=self.suppress if self.suppress_tail else None, ngen=self.ngen,
                                min_new=s.min_new_tokens, eos=self.eos, id0=self.id0, pos=self.pos))
            return
        nxt = _sample(self._process(self.logit_t), s.do_sample, s.temperature, s.top_k)
        self.next_id0.copy_(nxt)
        self.seen.scatter_(1, nxt, True)
        self.ngen.add_(1)
        self.pos.add_(1)
        self.id0.copy_(nxt)

    # --- prompt state -------------------------------------------------------------------------------------
    def load_kv(self, K: torch.Tensor, V: torch.Tensor) -> None:
        """Copies prior cache contents [layers, nkv, T, 128] into positions [0, T) (a prefilled prompt)."""
        T = K.shape[2]
        if T > self.max_cache:
            raise ValueError("prefill longer than the cache")
        self.kc[:, :, :T].copy_(K.to(self.kc.dtype))
        self.vc[:, :, :T].copy_(V.to(self.vc.dtype))

    def reset(self, pos: int, token: int) -> None:
        """Frame state right after a prompt of ``pos`` tokens whose first sampled code is ``token``
        (what the reference's _prefill_body leaves, qwen3/fast.py:253-263)."""
        self.id0.fill_(int(token))
        self.next_id0.fill_(int(token))
        self.seen.zero_()
        self.seen[0, int(token)] = True
        self.ngen.fill_(1)
        self.pos.fill_(int(pos))

    def _start(self, kw: dict) -> int:
        """Frame state after the prompt. With ``inputs_embeds`` (the reference's generate kwargs) the prompt runs
        through the talker's Hugging Face modules into the shared cache (``_prefill``: one recorded graph per prompt
        length, or eagerly without graphs); otherwise the prefill ran elsewhere and
        ``prefill_len``, ``first_token`` and, with a code predictor, ``last_hidden`` (the talker's last hidden state
        after its final norm, which the reference takes from the prefill, qwen3/kernels.py:678-679) give its
        results. ``tts_pad_embed`` as in qwen3/kernels.py:709."""
        if self.cp is not None and "tts_pad_embed" in kw:
            self.pad16.copy_(torch.as_tensor(kw["tts_pad_embed"]).reshape(-1).to(self.pad16))
        if "inputs_embeds" in kw:
            embeds = torch.as_tensor(kw["inputs_embeds"])
            self._check_prompt(embeds)
            self._prefill(embeds.to(device=self.device, dtype=self._prompt_dtype()))
            return int(embeds.shape[1])
        if self.cp is not None and "last_hidden" in kw:
            self.ph32.copy_(torch.as_tensor(kw["last_hidden"]).reshape(-1).to(self.ph32))
        L = int(kw["prefill_len"])
        self.reset(L, int(kw["first_token"]))
        return L

    def _prompt_dtype(self) -> torch.dtype:
        model = getattr(self.talker, "model", None)
        params = getattr(model, "parameters", None)
        p = next(params(), None) if callable(params) else None
        return p.dtype if p is not None else self.dtype

    def _check_prompt(self, embeds: torch.Tensor) -> None:
        if self.tcache is None:
            raise RuntimeError("prompt prefill needs the talker's runnable Hugging Face modules (tts.model.talker.model)")
        if embeds.dim() != 3 or embeds.shape[0] != 1:
            raise ValueError(f"inputs_embeds must be (1, L, H), got {tuple(embeds.shape)}")
        L = int(embeds.shape[1])
        if L < 1 or L >= self.max_cache:
            raise ValueError(f"prompt too long ({L} tokens, cache {self.max_cache})")

    def _prefill_body(self, embeds: torch.Tensor, cpos: torch.Tensor) -> None:
        """The prompt through the talker's Hugging Face modules into the shared cache (positions [0, L)), then what
        the reference's _prefill_body leaves (qwen3/fast.py:251-263 with _after_prefill, qwen3/kernels.py:695-703):
        the first code drawn from the codec head through the processor and the torch-path sampler, ``seen`` holding
        it, ``ngen`` 1, ``pos`` L, and the last hidden state (after the final norm) for the code predictor. Device
        work only, so it can be recorded in a graph."""
        self.seen.zero_()
        self.ngen.zero_()
        hidden = self._prefill_run(embeds, cpos)
        first = _sample(self._process(self._head_logits(hidden)), self.s.do_sample, self.s.temperature, self.s.top_k)
        self.id0.copy_(first)
        self.next_id0.copy_(first)
        self.ph32.copy_(hidden[0, -1].float())
        self.seen.scatter_(1, first, True)
        self.ngen.fill_(1)
        self.pos.fill_(int(embeds.shape[1]))

    def _head_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """fp32 (1, V) codec-head logits of the last position of ``hidden`` through the talker's own module."""
        head = self.talker.codec_head
        logits = head(hidden) if callable(head) else torch.nn.functional.linear(hidden, head.weight.to(hidden.dtype))
        return logits[:, -1, :].to(torch.float32)

    def _prefill_run(self, embeds: torch.Tensor, cpos: torch.Tensor | None = None) -> torch.Tensor:
        """The talker's Hugging Face modules over the prompt (1, L, H), writing its keys and values into positions
        [0, L) of the engine's cache through ``tcache``. Returns the last hidden state (after the final norm)."""
        L = int(embeds.shape[1])
        cpos = torch.arange(L, device=self.device) if cpos is None else cpos
        self.tcache.seek(0)
        out = self.talker.model(inputs_embeds=embeds, past_key_values=self.tcache, cache_position=cpos, use_cache=True)
        return out.last_hidden_state

    @torch.no_grad()
    def teacher_logits(self, kw: dict, codes: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Teacher forcing (qwen3/kernels.py:714-753): the prompt ``kw["inputs_embeds"]`` through the talker's
        Hugging Face modules, then for each frame f of ``codes`` (frames, G) the code predictor's positions fed the
        given codes (position 0 the talker's last hidden state, position 1 code 0 in the talker's table, position
        g >= 2 code g - 1 in table g - 2), the logits of heads 1..G-1, then the talker step on talker_in of the
        frame's codes at position L + f and its logits. Returns (talker logits (1 + frames, V), code-predictor
        logits (frames, G - 1, V_cp)), float32 on the CPU. Runs on the per-op kernels: the one-launch kernels pick
        their own codes. Draws no random numbers and leaves the frame state (``id0``, ``pos``, ``seen``) as the
        last frame put it, as the reference does."""
        if self.cp is None:
            raise ValueError("teacher_logits needs a code predictor")
        codes = torch.as_tensor(codes)
        if codes.dim() != 2 or codes.shape[1] != self.G:
            raise ValueError(f"codes must be (frames, {self.G}), got {tuple(codes.shape)}")
        if "tts_pad_embed" in kw:
            self.pad16.copy_(torch.as_tensor(kw["tts_pad_embed"]).reshape(-1).to(self.pad16))
        embeds = torch.as_tensor(kw["inputs_embeds"])
        self._check_prompt(embeds)
        L = int(embeds.shape[1])
        hidden = self._prefill_run(embeds.to(device=self.device, dtype=self._prompt_dtype()))
        if L + codes.shape[0] > self.max_cache:
            raise ValueError(f"prompt of {L} and {codes.shape[0]} frames exceed the cache ({self.max_cache})")
        l0 = [self._head_logits(hidden).cpu()]
        self.ph32.copy_(hidden[0, -1].float())
        P, lcp = self.C, []
        ck, cv = list(self.ck.unbind(0)), list(self.cv.unbind(0))
        cptr = self.codes.data_ptr()
        for f in range(codes.shape[0]):
            self.codes.copy_(codes[f].view(1, -1).to(self.codes))
            self.id0.copy_(self.codes[:, :1])
            frame = []
            for g in range(self.G):
                if g == 0:
                    self._cp_input(self.ph32)
                else:
                    self._embed(self.temb if g == 1 else self.cemb[g - 2], self.id0 if g == 1 else cptr + 8 * (g - 1),
                                self.e)
                    self._cp_input(self.e)
                self._layers(P, self.hc, self.qkv_c, self.att_c, self.act_c, ck, cv, None, g)
                if g > 0:
                    self._rms_gemv(self.hc, P.norm, P.eps, self.cp_heads[g - 1], self.logit_c, False)
                    frame.append(self.logit_c.clone().view(1, -1))
            self.pos.fill_(L + f)
            self._talker()  # talker_in of the frame's codes; the final norm's output lands in ph32
            lcp.append(torch.cat(frame, dim=0).cpu())
            l0.append(self.logit_t.clone().view(1, -1).cpu())
        return torch.cat(l0, dim=0), torch.stack(lcp, dim=0)

    @torch.no_grad()
    def layer_trace(self, token: int, pos: int) -> list[torch.Tensor]:
        """Runs one talker step eagerly and returns the residual after every layer, then the logits."""
        self.id0.fill_(int(token))
        self.pos.fill_(int(pos))
        self.trace = []
        try:
            self._talker()
            out = self.trace + [self.logit_t.clone()]
        finally:
            self.trace = None
        return out

    def generate_codes(self, kw: dict, max_frames: int | None = None) -> torch.Tensor:
        if self.fs is not None:
            # the fused sampler's key is drawn from torch's CPU generator, so torch.manual_seed reproduces a run and
            # successive calls differ (qwen3/kernels.py:709-713); the draw counter restarts at 0
            self.fs.set_seed(int(torch.randint(0, 2**62, (1,)).item()))
        return super().generate_codes(kw, max_frames=max_frames)

    def weight_bytes(self) -> dict:
        cp = self.C.bytes() if self.cp is not None else 0
        heads = sum(h.bytes() for h in self.cp_heads) if self.cp is not None else 0
        return {"talker": self.T.bytes() + self.codec_head.bytes(), "code_predictor": cp, "cp_heads": heads}
