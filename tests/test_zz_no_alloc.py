"""sk_attn_noalloc (the allocation-free variant of sk_attn, scratch in a static device array) against sk_attn on the
same inputs. Every cache here is longer than 128 positions, so each call splits the cache and merges the partials
through the shared arrival counters of the static scratch: three calls in a row (the second smaller, the third the
longest), then a refused position followed by a merged call, then replays of a captured call."""

import numpy as np
import pytest
import torch

from oracle import talker as O
from sokutou_amd import _lib
from sokutou_amd import synthetic as syn

pytestmark = pytest.mark.gpu
F32 = np.float32


def _case(gpu, rng, nkv, max_len, pos):
    nq = 2 * nkv
    K0 = torch.from_numpy(rng.standard_normal((nkv, max_len, 128)).astype(F32)).to(torch.bfloat16).to(gpu)
    V0 = torch.from_numpy(rng.standard_normal((nkv, max_len, 128)).astype(F32)).to(torch.bfloat16).to(gpu)
    qkv = torch.from_numpy(rng.standard_normal((nq + 2 * nkv) * 128).astype(F32)).to(gpu)
    qn = torch.from_numpy((1 + 0.1 * rng.standard_normal(128)).astype(F32)).to(gpu)
    kn = torch.from_numpy((1 + 0.1 * rng.standard_normal(128)).astype(F32)).to(gpu)
    rope = torch.from_numpy(O.rope_table(syn.inv_freq(syn.shape("0.6b")), max_len)).to(gpu)
    posg = torch.tensor([pos], dtype=torch.int64, device=gpu)
    return dict(nq=nq, nkv=nkv, max_len=max_len, K0=K0, V0=V0, qkv=qkv, qn=qn, kn=kn, rope=rope, pos=posg)


def _with_workspace(c, gpu):
    L, p = _lib.load(), _lib.ptr
    K, V = c["K0"].clone(), c["V0"].clone()
    out = torch.full((c["nq"] * 128,), 7.0, device=gpu)
    ws = torch.zeros(int(L.sk_attn_workspace_size(c["nq"], c["nkv"], c["max_len"])), dtype=torch.uint8, device=gpu)
    _lib.call("sk_attn", p(c["qkv"]), p(c["qn"]), p(c["kn"]), 1e-6, p(c["rope"]), p(K), p(V), p(c["pos"]), 0,
              c["max_len"], c["nq"], c["nkv"], p(out), p(ws), ws.numel(), 0, _lib.stream())
    torch.cuda.synchronize()
    assert int(ws[:4].view(torch.int32).item()) == 0
    return out, K, V


def _no_alloc(c, gpu, err):
    p = _lib.ptr
    K, V = c["K0"].clone(), c["V0"].clone()
    out = torch.full((c["nq"] * 128,), 7.0, device=gpu)
    _lib.call("sk_attn_noalloc", p(c["qkv"]), p(c["qn"]), p(c["kn"]), 1e-6, p(c["rope"]), p(K), p(V), p(c["pos"]), 0,
              c["max_len"], c["nq"], c["nkv"], p(out), p(err), 0, _lib.stream())
    torch.cuda.synchronize()
    return out, K, V


CASES = ((8, 577, 512), (4, 300, 200), (8, 2048, 2047))


def test_no_alloc_attention_matches_workspace_attention(gpu):
    print("sk_attn_noalloc: three merged calls in a row (nkv / max_len / pos " +
          ", ".join("%d / %d / %d" % c for c in CASES) + ") against sk_attn", flush=True)
    rng = np.random.default_rng(11)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    for nkv, max_len, pos in CASES:
        c = _case(gpu, rng, nkv, max_len, pos)
        want = _with_workspace(c, gpu)
        got = _no_alloc(c, gpu, err)
        assert int(err.item()) == 0
        # same kernel, same split and merge order: identical bits (output, appended K and V)
        for a, b in zip(got, want):
            assert torch.equal(a, b)
        assert not bool((got[0] == 7.0).any())


def test_no_alloc_attention_refuses_bad_position_then_runs(gpu):
    print("sk_attn_noalloc: position past the cache refused (err 5, nothing written), then a merged valid call",
          flush=True)
    rng = np.random.default_rng(12)
    c = _case(gpu, rng, 8, 577, 577)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    out, K, V = _no_alloc(c, gpu, err)
    assert int(err.item()) == 5
    assert bool((out == 7.0).all()) and torch.equal(K, c["K0"]) and torch.equal(V, c["V0"])
    err.zero_()
    c["pos"].fill_(540)  # 541 positions: split 8 ways and merged through the shared counters
    want = _with_workspace(c, gpu)
    got = _no_alloc(c, gpu, err)
    assert int(err.item()) == 0
    for a, b in zip(got, want):
        assert torch.equal(a, b)


def test_no_alloc_attention_replays_in_a_graph(gpu):
    """A call recorded into a graph (after the first call on the device, which sets the scratch up outside capture)
    replays with the counters of the static scratch back at zero each time: each replay equals sk_attn."""
    print("sk_attn_noalloc: a merged call captured in a graph, replayed three times against sk_attn", flush=True)
    rng = np.random.default_rng(13)
    c = _case(gpu, rng, 8, 577, 530)
    want = _with_workspace(c, gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    _no_alloc(c, gpu, err)  # the device's scratch is set up (a no-op if an earlier call did it)
    p = _lib.ptr
    K, V = c["K0"].clone(), c["V0"].clone()
    out = torch.full((c["nq"] * 128,), 7.0, device=gpu)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.call("sk_attn_noalloc", p(c["qkv"]), p(c["qn"]), p(c["kn"]), 1e-6, p(c["rope"]), p(K), p(V),
                  p(c["pos"]), 0, c["max_len"], c["nq"], c["nkv"], p(out), p(err), 0, _lib.stream())
    for _ in range(3):
        K.copy_(c["K0"])
        V.copy_(c["V0"])
        out.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        for a, b in zip((out, K, V), want):
            assert torch.equal(a, b)


def test_no_alloc_attention_rejects_too_many_heads_on_the_host(gpu):
    L = _lib.load()
    d = torch.zeros(64, device=gpu)
    p = d.data_ptr()
    rc = L.sk_attn_noalloc(p, p, p, 1e-6, p, p, p, None, 0, 64, 34, 17, p, None, 0, _lib.stream())
    assert rc == _lib.SK_EINVAL
