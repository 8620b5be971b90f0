"""Batched talker decode: up to 16 independent streams stepped together, each projection an M=16 GEMM on the
matrix cores (``sk_batch_frame``).

The reference decodes one stream at a time (qwen3/fast.py:146); this engine runs the same layer math as
``Qwen3Kernels`` (qwen3/kernels.py:619-627 per layer, then the final RMSNorm, the codec head and a greedy pick per
stream) for a batch whose streams sit at different positions, each with its own KV cache. The weights are the
talker's, quantised exactly as ``_Lin`` does (``i8row``) and rewritten once into the GEMM's tile layout.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .kernels import HD, _Lin, _Stack

MAX_BATCH = 16


def tile(lin: _Lin) -> torch.Tensor:
    """The int8 weights of ``lin`` in the batched GEMM's tile layout (``sk_tile_weights``)."""
    if lin.wd != "i8row":
        raise ValueError("the batched GEMM reads i8row weights")
    out = torch.empty_like(lin.w)
    _lib.call("sk_tile_weights", lin.w.data_ptr(), out.data_ptr(), lin.N, lin.K, _lib.stream())
    return out


class BatchedTalker:
    """``batch`` talker streams over one set of weights. State per stream: its KV cache (positions
    ``[0, max_len)``), its current token ``ids[b]``, its position ``pos[b]`` and the codes it has picked
    (``codes[f, b]``, ``nstep[b]`` of them).

    ``talker`` is the object ``Qwen3Kernels`` reads (``model.layers``, ``model.norm``, ``model.rotary_emb``,
    ``codec_head``, ``get_input_embeddings()``, qwen3/kernels.py:454-476, 516-523)."""

    def __init__(self, talker, batch: int, max_len: int, max_frames: int = 1024, device=None):
        if not 1 <= batch <= MAX_BATCH:
            raise ValueError(f"batch must be 1..{MAX_BATCH}")
        L = _lib.load()
        self.device = torch.device(device) if device is not None else talker.codec_head.weight.device
        if self.device.type != "cuda":
            raise RuntimeError("BatchedTalker runs on a HIP device")
        with torch.cuda.device(self.device):
            _lib.check(L.sk_device_check(), "sk_device_check")
        self.batch, self.max_len, self.max_frames = int(batch), int(max_len), int(max_frames)
        dev = self.device
        with torch.no_grad():
            P = _Stack(talker.model, "i8row", self.max_len)
            head = _Lin(talker.codec_head.weight, "i8row")
            for Ly in P.layers:
                for m in ("qkv", "o", "gu", "down"):
                    Ly[m].w = Ly[m].w.to(dev)
                    Ly[m].s = Ly[m].s.to(dev)
                    Ly[m].w = tile(Ly[m])
            head.w, head.s = head.w.to(dev), head.s.to(dev)
            head.w = tile(head)
            self.emb = talker.get_input_embeddings().weight.to(device=dev, dtype=torch.bfloat16).contiguous()
        for k in ("norm", "rope"):
            setattr(P, k, getattr(P, k).to(dev))
        for Ly in P.layers:
            for k in ("in_norm", "post_norm", "qn", "kn"):
                Ly[k] = Ly[k].to(dev)
        self.P, self.head = P, head
        self.V = head.N
        nl = len(P.layers)
        i64 = dict(dtype=torch.int64, device=dev)
        self.kc = torch.zeros((nl, self.batch, P.nkv, self.max_len, HD), dtype=torch.bfloat16, device=dev)
        self.vc = torch.zeros_like(self.kc)
        self.ids = torch.zeros(self.batch, **i64)
        self.pos = torch.zeros(self.batch, **i64)
        self.nstep = torch.zeros(self.batch, **i64)
        self.codes = torch.zeros((self.max_frames, MAX_BATCH), **i64)
        self.logits: torch.Tensor | None = None
        self.layer_out: torch.Tensor | None = None
        self.ws = torch.zeros(int(L.sk_batch_workspace_size(P.H, P.I, P.nq, P.nkv, self.V)), dtype=torch.uint8,
                              device=dev)
        arr = (_lib.SkLayerDesc * nl)()
        for i, Ly in enumerate(P.layers):
            arr[i] = _lib.SkLayerDesc(Ly["qkv"].w.data_ptr(), Ly["qkv"].s.data_ptr(), Ly["o"].w.data_ptr(),
                                      Ly["o"].s.data_ptr(), Ly["gu"].w.data_ptr(), Ly["gu"].s.data_ptr(),
                                      Ly["down"].w.data_ptr(), Ly["down"].s.data_ptr(), Ly["in_norm"].data_ptr(),
                                      Ly["post_norm"].data_ptr(), Ly["qn"].data_ptr(), Ly["kn"].data_ptr(),
                                      self.kc[i].data_ptr(), self.vc[i].data_ptr())
        self._layers = arr  # host array read by sk_batch_frame at every call
        self._desc = _lib.SkBatchDesc(
            n_layers=nl, hidden=P.H, inter=P.I, nq=P.nq, nkv=P.nkv, vocab=self.V, batch=self.batch,
            max_len=self.max_len, eps=P.eps, layers=ctypes.cast(arr, ctypes.c_void_p), norm=P.norm.data_ptr(),
            head_w=head.w.data_ptr(), head_s=head.s.data_ptr(), emb=self.emb.data_ptr(), rope=P.rope.data_ptr(),
            ids=self.ids.data_ptr(), pos=self.pos.data_ptr(), codes=self.codes.data_ptr(),
            nstep=self.nstep.data_ptr(), max_frames=self.max_frames, logits=None, layer_out=None,
            workspace=self.ws.data_ptr(), workspace_bytes=self.ws.numel())
        self.graph: torch.cuda.CUDAGraph | None = None

    # --- state -----------------------------------------------------------------------------------------------
    def load_kv(self, b: int, K: torch.Tensor, V: torch.Tensor) -> None:
        """Prior cache of stream ``b``: [layers, nkv, T, 128] into positions [0, T)."""
        T = K.shape[2]
        if T > self.max_len:
            raise ValueError("prefill longer than the cache")
        self.kc[:, b, :, :T].copy_(K.to(self.kc.dtype))
        self.vc[:, b, :, :T].copy_(V.to(self.vc.dtype))

    def reset(self, pos, tokens) -> None:
        """Stream b continues at position ``pos[b]`` with input token ``tokens[b]``; the code record restarts."""
        if len(pos) != self.batch or len(tokens) != self.batch:
            raise ValueError("one position and one token per stream")
        if any(not 0 <= int(p) < self.max_len for p in pos) or any(not 0 <= int(t) < self.V for t in tokens):
            raise ValueError("position or token out of range")
        self.pos.copy_(torch.tensor([int(p) for p in pos], dtype=torch.int64))
        self.ids.copy_(torch.tensor([int(t) for t in tokens], dtype=torch.int64))
        self.nstep.zero_()
        self.ws[:4].zero_()
        _lib.check(_lib.load().sk_batch_embed(ctypes.byref(self._desc), _lib.stream()), "sk_batch_embed")

    # --- steps -----------------------------------------------------------------------------------------------
    def step(self) -> None:
        """One decode step of every stream on the current stream (6 launches per layer: qkv, attention, its merge,
        o, gate/up, down; then the head and the pick)."""
        self._desc.logits = None if self.logits is None else self.logits.data_ptr()
        self._desc.layer_out = None if self.layer_out is None else self.layer_out.data_ptr()
        _lib.check(_lib.load().sk_batch_frame(ctypes.byref(self._desc), _lib.stream()), "sk_batch_frame")

    def capture(self) -> None:
        """Records one step as a HIP graph. One eager warm-up step runs first on a side stream (first-use set-up
        stays out of the graph); then positions, tokens, pick counts and the error word are restored and the inputs
        re-embedded from the restored tokens, so capturing leaves the streams where they were (the warm-up's cache
        row at each stream's position is rewritten by the next step)."""
        saved = [t.clone() for t in (self.pos, self.ids, self.nstep)]
        err = self.ws[:4].clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step()
        torch.cuda.current_stream().wait_stream(side)
        for t, v in zip((self.pos, self.ids, self.nstep), saved):
            t.copy_(v)
        self.ws[:4].copy_(err)
        _lib.check(_lib.load().sk_batch_embed(ctypes.byref(self._desc), _lib.stream()), "sk_batch_embed")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        self.graph = g

    def replay(self, n: int = 1) -> None:
        for _ in range(n):
            if self.graph is not None:
                self.graph.replay()
            else:
                self.step()

    def error(self) -> int:
        """Error word (0 healthy; 5 a position or token out of range, 6 more picks than ``max_frames``)."""
        return int(self.ws[:4].view(torch.int32).item())

    def picked(self) -> torch.Tensor:
        """[n, batch] codes picked so far (n = the smallest pick count over the streams)."""
        n = int(self.nstep.min().item())
        return self.codes[:n, : self.batch]

    def weight_bytes(self) -> int:
        return self.P.bytes() + self.head.bytes()
