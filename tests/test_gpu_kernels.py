"""Per-kernel parity of the HIP path (through the C-ABI) against the CPU oracle on the same seeded inputs."""

import numpy as np
import pytest
import torch

from oracle import talker as O
from sokutou_amd import _lib
from sokutou_amd import synthetic as syn
from sokutou_amd.kernels import _Lin

pytestmark = pytest.mark.gpu
F32 = np.float32

# GEMV shapes of one layer at 0.6B and 1.7B (qkv, o, gate/up, down) and the codec head
SHAPES = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072), (3072, 1024), (4096, 2048), (2048, 6144), (512, 512),
          (1030, 1024), (18, 2048)]


def rel_err(a, b) -> float:
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else a
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


@pytest.mark.parametrize("wd", ["i8row", "i8g32", "bf16", "f32"])
@pytest.mark.parametrize("N,K", SHAPES)
def test_gemv_family(gpu, wd, N, K):
    print(f"gemv wd={wd} N={N} K={K}", flush=True)
    rng = np.random.default_rng(N * 7 + K)
    w = (rng.standard_normal((N, K)) * 0.02).astype(F32)
    qo, so, deq = O.quantize(w, wd)
    lin = _Lin(_t(w, gpu), wd)
    if so is not None:  # the packed weights on the device are the oracle's, bit for bit
        assert np.array_equal(lin.w.cpu().numpy(), qo)
        assert np.array_equal(lin.s.cpu().numpy().view(np.uint16), so)
    x = rng.standard_normal(K).astype(F32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(F32)
    bias = rng.standard_normal(N).astype(F32)
    base = rng.standard_normal(N).astype(F32)
    p = _lib.ptr
    st = _lib.stream()
    code = _lib.WD[wd]
    xg, nwg, bg = _t(x, gpu), _t(nw, gpu), _t(bias, gpu)
    for pol in (0, 1):
        out = torch.zeros(N, device=gpu)
        _lib.call("sk_gemv", p(xg), p(lin.w), p(lin.s), None, p(out), N, K, 0, code, pol, st)
        torch.cuda.synchronize()
        assert rel_err(out, O.gemv(x, deq)) < 1e-5
        out = _t(base, gpu)
        _lib.call("sk_gemv", p(xg), p(lin.w), p(lin.s), p(bg), p(out), N, K, 1, code, pol, st)
        torch.cuda.synchronize()
        assert rel_err(out, O.gemv(x, deq, bias, base)) < 1e-5
        out = torch.zeros(N, device=gpu)
        _lib.call("sk_rms_gemv", p(xg), p(nwg), 1e-6, p(lin.w), p(lin.s), p(out), N, K, 0, code, pol, st)
        torch.cuda.synchronize()
        assert rel_err(out, O.rms_gemv(x, nw, 1e-6, deq)) < 1e-5
        out = torch.zeros(N // 2, device=gpu)
        _lib.call("sk_rms_gemv", p(xg), p(nwg), 1e-6, p(lin.w), p(lin.s), p(out), N, K, 1, code, pol, st)
        torch.cuda.synchronize()
        assert rel_err(out, O.rms_gemv(x, nw, 1e-6, deq, swiglu=True)) < 1e-5


def _attn_case(gpu, seed, nkv, max_len, pos, ct):
    nq = 2 * nkv
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal((nq + 2 * nkv) * 128).astype(F32)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(F32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(F32)
    Kc = rng.standard_normal((nkv, max_len, 128)).astype(F32)
    Vc = rng.standard_normal((nkv, max_len, 128)).astype(F32)
    if ct == "bf16":
        Kc, Vc = O.bf16_round(Kc), O.bf16_round(Vc)
    rope = O.rope_table(syn.inv_freq(syn.shape("0.6b")), max_len)
    dt = torch.bfloat16 if ct == "bf16" else torch.float32
    Kg, Vg = _t(Kc, gpu).to(dt), _t(Vc, gpu).to(dt)
    L = _lib.load()
    ws = torch.zeros(int(L.sk_attn_workspace_size(nq, nkv, max_len)), dtype=torch.uint8, device=gpu)
    out = torch.zeros(nq * 128, device=gpu)
    posg = torch.tensor([pos - 3], dtype=torch.int64, device=gpu)
    p = _lib.ptr
    qkvg, qng, kng, ropeg = _t(qkv, gpu), _t(qn, gpu), _t(kn, gpu), _t(rope, gpu)
    for _ in range(2):  # twice: the arrival counters must come back to zero
        _lib.call("sk_attn", p(qkvg), p(qng), p(kng), 1e-6, p(ropeg), p(Kg), p(Vg), p(posg), 3, max_len, nq, nkv, p(out),
                  p(ws), ws.numel(), _lib.CT[ct], _lib.stream())
    torch.cuda.synchronize()
    Ko, Vo = Kc.copy(), Vc.copy()
    ref = O.attention(qkv, qn, kn, 1e-6, rope, Ko, Vo, pos, nq, nkv, cache_bf16=(ct == "bf16"))
    return out, ref, Kg.float().cpu().numpy(), Vg.float().cpu().numpy(), Ko, Vo, ws


@pytest.mark.parametrize("ct", ["bf16", "f32"])
@pytest.mark.parametrize("nkv,max_len,pos", [(8, 1024, 0), (8, 1024, 1), (8, 1024, 16), (8, 1024, 256), (8, 1024, 512),
                                             (8, 1024, 575), (8, 1024, 1023), (8, 576, 575), (8, 16, 15), (8, 16, 3),
                                             (2, 64, 40), (8, 2048, 2047), (8, 1024, 63), (8, 1024, 64), (8, 129, 128),
                                             (8, 4096, 1000), (8, 4096, 4095)])
def test_attention(gpu, ct, nkv, max_len, pos):
    print(f"attn ct={ct} nkv={nkv} max_len={max_len} pos={pos}", flush=True)
    out, ref, Kg, Vg, Ko, Vo, ws = _attn_case(gpu, pos + 31 * nkv, nkv, max_len, pos, ct)
    assert rel_err(out, ref) < 2e-5
    # the appended entry: the same bf16 value, or one bf16 step away where fp32 rounding straddles a tie
    dk = np.abs(Kg[:, pos] - Ko[:, pos])
    if ct == "bf16":
        step = np.abs(Ko[:, pos]) * 2.0 ** -7 + 1e-30
        assert np.all(dk <= step) and np.mean(dk > 0) < 0.02
    else:
        np.testing.assert_allclose(Kg[:, pos], Ko[:, pos], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(Vg[:, pos], Vo[:, pos])
    # nothing else in the cache changed
    mask = np.ones(max_len, bool)
    mask[pos] = False
    np.testing.assert_array_equal(Kg[:, mask], Ko[:, mask])
    np.testing.assert_array_equal(Vg[:, mask], Vo[:, mask])
    # the error word (bytes 0..3) is clear and every head's arrival counter (from byte 4) is back at zero
    assert int(ws[:4].view(torch.int32).item()) == 0
    assert int(ws[4 : 4 + 4 * nkv].view(torch.int32).abs().sum()) == 0


def test_attention_invalid_position_sets_error_word(gpu):
    nkv, max_len = 8, 64
    rng = np.random.default_rng(5)
    Kg = torch.zeros((nkv, max_len, 128), dtype=torch.bfloat16, device=gpu)
    Vg = torch.zeros_like(Kg)
    qkv = _t(rng.standard_normal(32 * 128).astype(F32), gpu)
    ones = torch.ones(128, device=gpu)
    rope = _t(O.rope_table(syn.inv_freq(syn.shape("0.6b")), max_len), gpu)
    L = _lib.load()
    ws = torch.zeros(int(L.sk_attn_workspace_size(16, nkv, max_len)), dtype=torch.uint8, device=gpu)
    out = torch.full((16 * 128,), 7.0, device=gpu)
    posg = torch.tensor([max_len], dtype=torch.int64, device=gpu)
    p = _lib.ptr
    _lib.call("sk_attn", p(qkv), p(ones), p(ones), 1e-6, p(rope), p(Kg), p(Vg), p(posg), 0, max_len, 16, nkv, p(out),
              p(ws), ws.numel(), 0, _lib.stream())
    torch.cuda.synchronize()
    # refused on the device: error word 5, caches and output untouched
    assert int(ws[:4].view(torch.int32).item()) == 5
    assert float(Kg.abs().sum()) == 0 and float(Vg.abs().sum()) == 0
    assert bool((out == 7.0).all())
    # the arrival counters are still zero: a later valid call on the same workspace (error word cleared) merges
    ws[:4].zero_()
    posg.fill_(3)
    _lib.call("sk_attn", p(qkv), p(ones), p(ones), 1e-6, p(rope), p(Kg), p(Vg), p(posg), 0, max_len, 16, nkv, p(out),
              p(ws), ws.numel(), 0, _lib.stream())
    torch.cuda.synchronize()
    assert int(ws[:4].view(torch.int32).item()) == 0
    assert int(ws[4:4 + 4 * nkv].view(torch.int32).abs().sum().item()) == 0
    assert bool(torch.isfinite(out).all()) and not bool((out == 7.0).any())


def test_rmsnorm_embed(gpu):
    rng = np.random.default_rng(9)
    for K in (1024, 2048, 100):
        h = rng.standard_normal(K).astype(F32)
        nw = (1 + 0.1 * rng.standard_normal(K)).astype(F32)
        out = torch.zeros(K, device=gpu)
        hg, nwg = _t(h, gpu), _t(nw, gpu)  # keep the tensors alive until the kernel has run
        _lib.call("sk_rmsnorm", _lib.ptr(hg), _lib.ptr(nwg), 1e-6, _lib.ptr(out), K, _lib.stream())
        torch.cuda.synchronize()
        assert rel_err(out, O.rmsnorm(h, nw, 1e-6)) < 2e-6
    tab = syn.bf16_values(rng.standard_normal((50, 1024)).astype(F32))
    tg = _t(tab, gpu).to(torch.bfloat16)
    out = torch.zeros(1024, device=gpu)
    idx = torch.tensor([37], dtype=torch.int64, device=gpu)
    _lib.call("sk_embed", _lib.ptr(tg), _lib.ptr(idx), _lib.ptr(out), 1024, 0, _lib.stream())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), tab[37])


def test_talker_in(gpu):
    rng = np.random.default_rng(10)
    G, dim = 4, 1024
    tabs = [syn.bf16_values(rng.standard_normal((30, dim)).astype(F32)) for _ in range(G)]
    pad = syn.bf16_values(rng.standard_normal(dim).astype(F32))
    tg = [_t(t, gpu).to(torch.bfloat16) for t in tabs]
    addr = torch.tensor([t.data_ptr() for t in tg], dtype=torch.int64, device=gpu)
    codes = torch.tensor([3, 29, 0, 11], dtype=torch.int64, device=gpu)
    out = torch.zeros(dim, device=gpu)
    padg = _t(pad, gpu).to(torch.bfloat16)
    _lib.call("sk_talker_in", _lib.ptr(addr), _lib.ptr(codes), _lib.ptr(padg), _lib.ptr(out), dim, G, 0, _lib.stream())
    torch.cuda.synchronize()
    ref = np.zeros(dim, F32)
    for g, c in enumerate([3, 29, 0, 11]):
        ref = ref + tabs[g][c]
    np.testing.assert_allclose(out.cpu().numpy(), ref + pad, rtol=1e-6, atol=1e-6)


def test_greedy_sampler_matches_oracle_2000_trials(gpu):
    """Known-answer check in the style of qwen3/check_sampler.py:41-64: processor + argmax + state update."""
    from sokutou_amd.sampler import FusedSampler

    fs = FusedSampler(gpu)
    rng = np.random.default_rng(0)
    V, eos = 3072, 2150
    sup = np.zeros(V, bool)
    sup[V - 1024:] = True
    sup[eos] = False
    supg = _t(sup, gpu)
    out = torch.zeros(1, dtype=torch.int64, device=gpu)
    bad = 0
    for trial in range(2000):
        lg = (rng.standard_normal(V) * 3).astype(F32)
        if trial % 3 == 0:
            lg[eos] = lg.max() + 1
        if trial % 7 == 0:  # exact ties: the lowest index must win
            j = int(rng.integers(0, 2000))
            lg[j + 1] = lg[j] = lg.max() + 0.5
        if trial % 11 == 0:
            lg[rng.integers(0, V, 20)] = np.nan
        seen = rng.random(V) < 0.05
        ngen_v = trial % 4
        ref = O.argmax_first(O.process_logits(lg, seen, 1.05, sup, ngen_v, 2, eos))
        seen_g = _t(seen, gpu)
        ngen = torch.tensor([ngen_v], dtype=torch.int64, device=gpu)
        id0 = torch.zeros(1, dtype=torch.int64, device=gpu)
        pos = torch.zeros(1, dtype=torch.int64, device=gpu)
        lgg = _t(lg, gpu)
        fs(lgg, out, False, 1.0, 0, talker=dict(seen=seen_g, rep_pen=1.05, suppress=supg, ngen=ngen, min_new=2,
                                                          eos=eos, id0=id0, pos=pos))
        torch.cuda.synchronize()
        s2 = seen_g.cpu().numpy()
        ok = (int(out) == ref and int(id0) == ref and int(ngen) == ngen_v + 1 and int(pos) == 1 and s2[ref]
              and int(s2.sum()) == int(seen.sum()) + (0 if seen[ref] else 1))
        bad += not ok
    assert bad == 0, f"{bad} of 2000 trials differ"


def test_plain_argmax_without_processor(gpu):
    from sokutou_amd.sampler import FusedSampler

    fs = FusedSampler(gpu)
    out = torch.zeros(1, dtype=torch.int64, device=gpu)
    for V in (1, 2, 2048, 3072, 4096):
        lg = np.random.default_rng(V).standard_normal(V).astype(F32)
        lgg = _t(lg, gpu)
        fs(lgg, out, False, 1.0, 0)
        torch.cuda.synchronize()
        assert int(out) == O.argmax_first(lg)
    lgg = _t(np.full(100, -np.inf, F32), gpu)
    fs(lgg, out, False, 1.0, 0)
    torch.cuda.synchronize()
    assert int(out) == 0


def _near_tie(g, pick, ref, rel=1e-5) -> bool:
    """True when the GPU's pick and the oracle's are within float rounding of each other (fp32 log on two devices)."""
    a, b = float(g[pick]), float(g[ref])
    return np.isfinite(a) and np.isfinite(b) and abs(a - b) <= rel * max(1.0, abs(b))


def test_sampled_picks_match_oracle(gpu):
    """do_sample = 1: processor, temperature, top-k threshold and the Gumbel-max draw from Philox4x32-10 give the
    oracle's pick for the same seed and counter (qwen3/sampler.py:37-159); the counter advances once per draw."""
    from sokutou_amd.sampler import FusedSampler

    fs = FusedSampler(gpu)
    seed = 0x1234_5678_9ABC
    fs.set_seed(seed)
    rng = np.random.default_rng(7)
    out = torch.zeros(1, dtype=torch.int64, device=gpu)
    bad, ties, n = [], 0, 1200
    eos = 2150
    for trial in range(n):
        V = (3072, 2048, 4096, 97, 1, 3072)[trial % 6]
        top_k = (0, 1, 50, V - 1, V, 2 * V, 17)[trial % 7]
        T = (0.7, 1.0, 1.3, 0.05)[trial % 4]
        lg = (rng.standard_normal(V) * 2).astype(F32)
        if trial % 5 == 0 and V > 10:  # ties around the threshold, -inf entries
            lg[rng.integers(0, V, 30)] = lg.max()
            lg[rng.integers(0, V, 5)] = -np.inf
        if trial % 13 == 0 and V > 10:
            lg[rng.integers(0, V, 3)] = np.nan
        talker = trial % 3 == 0 and V == 3072
        lgg = _t(lg, gpu)
        if talker:
            seen = rng.random(V) < 0.05
            sup = np.zeros(V, bool)
            sup[V - 1024:] = True
            ngen_v = trial % 4
            proc = O.process_logits(lg, seen, 1.05, sup, ngen_v, 2, eos)
            ngen = torch.tensor([ngen_v], dtype=torch.int64, device=gpu)
            fs(lgg, out, True, T, top_k, talker=dict(seen=_t(seen, gpu), rep_pen=1.05, suppress=_t(sup, gpu), ngen=ngen,
                                                     min_new=2, eos=eos, id0=None, pos=None))
        else:
            proc = lg
            fs(lgg, out, True, T, top_k)
        torch.cuda.synchronize()
        ref, g = O.sample_draw(proc, float(np.float32(1.0 / T)), top_k, seed, trial, exact=True)
        pick = int(out)
        if pick != ref:
            if _near_tie(g, pick, ref):
                ties += 1
            else:
                bad.append((trial, V, top_k, T, pick, ref))
    assert int(fs.counter) == n
    print(f"  {n} draws: {n - len(bad) - ties} identical, {ties} within rounding of a tie", flush=True)
    assert not bad, bad[:5]
    assert ties <= 2


def test_sampled_pick_replays_from_a_graph(gpu):
    """The draw counter lives in device memory: every replay of a captured pick draws the next number."""
    from sokutou_amd.sampler import FusedSampler

    fs = FusedSampler(gpu)
    fs.set_seed(99)
    V, top_k, T = 3072, 50, 0.9
    lg = (np.random.default_rng(3).standard_normal(V) * 2).astype(F32)
    lgg = _t(lg, gpu)
    out = torch.zeros(1, dtype=torch.int64, device=gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fs(lgg, out, True, T, top_k)  # counter 0
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fs(lgg, out, True, T, top_k)
    torch.cuda.synchronize()
    picks = []
    for _ in range(40):
        g.replay()
        torch.cuda.synchronize()
        picks.append(int(out))
    ref = [O.sample_draw(lg, float(np.float32(1.0 / T)), top_k, 99, c)[0] for c in range(1, 41)]
    assert picks == ref
    assert int(fs.counter) == 41 and len(set(picks)) > 5


def test_attention_workspace_shared_across_cache_lengths(gpu):
    """One workspace for attention over caches of different lengths (a talker and its code predictor): the
    counters sit at a fixed place, so a long call's partials never corrupt a short call's counters."""
    nkv, nq = 8, 16
    L = _lib.load()
    ws = torch.zeros(int(L.sk_attn_workspace_size(nq, nkv, 1024)), dtype=torch.uint8, device=gpu)
    rng = np.random.default_rng(12)
    rope_np = O.rope_table(np.float32(1.0) / (1e6 ** (np.arange(0, 128, 2) / 128)).astype(np.float32), 1024)
    rope = torch.from_numpy(rope_np).to(gpu)
    qn = torch.from_numpy((1 + 0.1 * rng.standard_normal(128)).astype(F32)).to(gpu)
    kn = torch.from_numpy((1 + 0.1 * rng.standard_normal(128)).astype(F32)).to(gpu)
    for max_len, pos in ((1024, 700), (16, 9), (1024, 300), (16, 15), (80, 50), (16, 3)):
        Kc = torch.from_numpy(O.bf16_round(rng.standard_normal((nkv, max_len, 128)).astype(F32))).to(gpu).to(torch.bfloat16)
        Vc = torch.from_numpy(O.bf16_round(rng.standard_normal((nkv, max_len, 128)).astype(F32))).to(gpu).to(torch.bfloat16)
        qkv = rng.standard_normal((nq + 2 * nkv) * 128).astype(F32)
        Kr, Vr = Kc.float().cpu().numpy().copy(), Vc.float().cpu().numpy().copy()
        ref = O.attention(qkv, qn.cpu().numpy(), kn.cpu().numpy(), 1e-6, rope_np, Kr, Vr, pos, nq, nkv)
        out = torch.zeros(nq * 128, device=gpu)
        p = _lib.ptr
        _lib.call("sk_attn", p(torch.from_numpy(qkv).to(gpu)), p(qn), p(kn), 1e-6, p(rope), p(Kc), p(Vc), None, pos,
                  max_len, nq, nkv, p(out), p(ws), ws.numel(), 0, _lib.stream())
        torch.cuda.synchronize()
        assert rel_err(out, ref) < 1e-5, (max_len, pos)
