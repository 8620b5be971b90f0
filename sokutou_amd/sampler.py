"""One-launch sampling step on the device (``sk_sample``), with the talker processor and the device-side state
update, so a whole frame can be replayed from a graph without a host round trip.

Mirrors ``FusedSampler`` of the reference (qwen3/sampler.py:165-191): greedy (``do_sample=False``, lowest index
on ties) or sampled (temperature, top-k threshold by radix select, Gumbel-max with Philox4x32-10 keyed by ``seed``
and counted by ``counter``). The same seed and counter give the reference kernel's pick; the counter advances on
the device, so each replay of a captured graph draws a new number.
"""

from __future__ import annotations

import torch

from . import _lib

MAX_V = 4096


class FusedSampler:
    """Launches the sampling kernel. ``seed`` and ``counter`` live in device memory (int64, one element each)."""

    def __init__(self, device):
        _lib.load()
        self.seed = torch.zeros(1, dtype=torch.int64, device=device)
        self.counter = torch.zeros(1, dtype=torch.int64, device=device)

    def set_seed(self, seed: int) -> None:
        self.seed.fill_(int(seed) & 0x7FFFFFFFFFFFFFFF)
        self.counter.zero_()

    def __call__(self, logits: torch.Tensor, out, do_sample: bool, temperature: float, top_k: int,
                 talker: dict | None = None) -> None:
        """Picks one id from ``logits`` (fp32, V <= 4096, contiguous) into ``out`` (int64 tensor or its address).
        ``talker`` (talker frames only) holds seen, rep_pen, suppress, ngen, min_new, eos, id0, pos."""
        V = logits.numel()
        if V > MAX_V or logits.dtype != torch.float32 or not logits.is_contiguous():
            raise ValueError("logits must be fp32, contiguous, with at most 4096 entries")
        tk = talker or {}
        p = _lib.ptr
        _lib.call("sk_sample", p(logits), V, 1.0 / temperature if do_sample else 1.0, int(top_k or 0), int(bool(do_sample)),
                  p(tk.get("seen")), float(tk.get("rep_pen", 1.0)), p(tk.get("suppress")), p(tk.get("ngen")),
                  int(tk.get("min_new", 0)), int(tk.get("eos", -1)), p(self.seed), p(self.counter), p(out),
                  int(talker is not None), p(tk.get("id0")), p(tk.get("pos")), _lib.stream())
