"""Pins the CPU oracle (oracle/talker.py) against independent references: torch's bf16 conversion, brute-force
loops, float64 closed forms and transformers' Qwen3 layer (a library implementation of the same architecture).
CPU only."""

import numpy as np
import pytest
import torch

from oracle import talker as O
from sokutou_amd import synthetic as syn

F32 = np.float32


# ---- bf16 storage rounding ----------------------------------------------------------------------------------
def test_bf16_matches_torch_on_all_classes():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(F32) * F32(3.0),
        rng.standard_normal(1000).astype(F32) * F32(1e-38),  # subnormals
        np.array([0.0, -0.0, np.inf, -np.inf, 1.0, -1.0, 3.4e38, -3.4e38, 1e-45], dtype=F32),
        # exact ties between two bf16 values, both parities of the kept bit
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(F32),
    ])
    got = O.bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_nan_rule():
    x = np.array([np.nan, -np.nan], dtype=F32)
    x = np.concatenate([x, np.array([0x7F800001, 0xFFC00001, 0x7FFFFFFF], dtype=np.uint32).view(F32)])
    assert np.all(O.bf16_bits(x) == 0x7FC0)


# ---- quantisation -------------------------------------------------------------------------------------------
def _brute_rowwise(w):
    N, K = w.shape
    q = np.zeros((N, K), np.int8)
    s_bits = np.zeros(N, np.uint16)
    for n in range(N):
        amax = F32(0)
        for k in range(K):
            amax = max(amax, abs(w[n, k]))
        s = F32(max(F32(amax / F32(127)), F32(1e-12)))
        sb = int(torch.tensor([float(s)], dtype=torch.float32).to(torch.bfloat16).view(torch.int16).item()) & 0xFFFF
        s_bits[n] = sb
        sv = np.array([sb << 16], np.uint32).view(F32)[0]
        for k in range(K):
            r = F32(w[n, k] / sv)
            # round half to even by hand
            f = np.floor(r)
            d = r - f
            v = f + 1 if d > 0.5 or (d == 0.5 and int(f) % 2 == 1) else f
            q[n, k] = int(min(127, max(-127, v)))
    return q, s_bits


def test_quantize_rowwise_brute_force():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((6, 64)) * 0.02).astype(F32)
    w[1] = 0.0  # all-zero row -> scale clamps to 1e-12, q = 0
    w[2, :4] = [F32(127 * 0.001), F32(-0.0005), F32(0.0015), F32(0.0025)]  # ties after division
    q, s = O.quantize_rowwise(w)
    qb, sb = _brute_rowwise(w)
    assert np.array_equal(s, sb)
    assert np.array_equal(q, qb)
    assert np.all(q[1] == 0)


def test_quantize_rowwise_ties_round_to_even():
    # scale exactly 1.0 (max 127): w/s lands on .5 ties
    w = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5] + [0.0] * 56], dtype=F32)
    q, s = O.quantize_rowwise(w)
    assert O.bf16_to_f32(s)[0] == 1.0
    assert list(q[0, :8]) == [127, 0, 2, 2, 0, -2, -2, 4]


def test_quantize_rowwise_clamps_when_scale_rounds_down():
    # max|w|/127 rounds down in bf16 -> the max element exceeds 127 * s and clamps to 127
    amax = F32(1.0) + F32(2 ** -12)
    w = np.zeros((1, 512), F32)
    w[0, 0] = amax
    w[0, 1] = -amax
    q, s = O.quantize_rowwise(w)
    assert q[0, 0] == 127 and q[0, 1] == -127


def test_quantize_g32_matches_brute_force():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((4, 128)) * 0.05).astype(F32)
    w[0, :32] = 0.0  # zero group -> fp16 scale underflows to 0, defined q = 0
    q, s = O.quantize_g32(w)
    for n in range(4):
        for gi in range(4):
            g = w[n, 32 * gi:32 * gi + 32]
            sc = np.float16(max(F32(np.abs(g).max() / F32(127)), F32(1e-12)))
            assert s[n, gi] == np.array([sc], np.float16).view(np.uint16)[0]
            for k in range(32):
                if float(sc) == 0.0:
                    expect = 0
                else:
                    expect = int(np.clip(np.rint(F32(g[k] / F32(sc))), -127, 127))
                assert q[n, 32 * gi + k] == expect
    assert np.all(q[0, :32] == 0)


@pytest.mark.parametrize("wd", ["i8row", "i8g32", "bf16", "f32"])
def test_lin_quantisation_matches_oracle_bit_exact(wd):
    from sokutou_amd.kernels import _Lin

    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 1024)) * 0.02).astype(F32)
    w[5] = 0.0
    lin = _Lin(torch.from_numpy(w), wd)
    qo, so, deq = O.quantize(w, wd)
    if wd in ("i8row", "i8g32"):
        assert np.array_equal(lin.w.numpy(), qo)
        assert np.array_equal(lin.s.numpy().view(np.uint16), so)
    elif wd == "bf16":
        assert np.array_equal(lin.w.view(torch.int16).numpy().view(np.uint16), qo)
    else:
        assert np.array_equal(lin.w.numpy(), qo)
    assert np.array_equal(lin.dequant().numpy(), deq)


def test_dequant_exact_in_fp32():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((8, 512)) * 0.02).astype(F32)
    q, s = O.quantize_rowwise(w)
    d64 = q.astype(np.float64) * O.bf16_to_f32(s).astype(np.float64)[:, None]
    assert np.array_equal(O.dequant_rowwise(q, s).astype(np.float64), d64)


# ---- RoPE table, norms, GEMV ----------------------------------------------------------------------------------
def test_rope_table_closed_form_and_hf_inv_freq():
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    s = syn.shape("0.6b")
    inv = syn.inv_freq(s)
    cfg = Qwen3Config(hidden_size=1024, num_attention_heads=16, num_key_value_heads=8, head_dim=128,
                      rope_parameters={"rope_type": "default", "rope_theta": 1e6})
    hf_inv, scaling = Qwen3RotaryEmbedding.compute_default_rope_parameters(cfg)
    assert scaling == 1.0 and np.array_equal(hf_inv.numpy(), inv)
    tab = O.rope_table(inv, 600)
    f = (np.arange(600, dtype=F32)[:, None] * inv[None, :]).astype(np.float64)
    assert np.array_equal(tab[:, :64], np.cos(f).astype(F32))
    assert np.array_equal(tab[:, 64:], np.sin(f).astype(F32))
    # the engine's torch table agrees to 2 ulp
    ft = torch.arange(600, dtype=torch.float32)[:, None] * torch.from_numpy(inv)[None, :]
    tt = torch.cat([ft.cos(), ft.sin()], 1).numpy()
    assert np.max(np.abs(tt - tab)) <= 2 * np.spacing(F32(1.0))


def test_rmsnorm_and_rms_gemv_against_float64():
    rng = np.random.default_rng(5)
    K, N = 512, 64
    h = rng.standard_normal(K).astype(F32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(F32)
    W = (rng.standard_normal((N, K)) * 0.02).astype(F32)
    h64, nw64, W64 = h.astype(np.float64), nw.astype(np.float64), W.astype(np.float64)
    inv = 1 / np.sqrt(np.mean(h64 ** 2) + 1e-6)
    np.testing.assert_allclose(O.rmsnorm(h, nw, 1e-6), h64 * inv * nw64, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(O.rms_gemv(h, nw, 1e-6, W), W64 @ (h64 * nw64) * inv, rtol=1e-5, atol=1e-6)
    y = W64 @ (h64 * nw64) * inv
    g, u = y[0::2], y[1::2]
    np.testing.assert_allclose(O.rms_gemv(h, nw, 1e-6, W, swiglu=True), g / (1 + np.exp(-g)) * u, rtol=1e-5, atol=1e-6)
    x = rng.standard_normal(K).astype(F32)
    b = rng.standard_normal(N).astype(F32)
    acc = rng.standard_normal(N).astype(F32)
    np.testing.assert_allclose(O.gemv(x, W, b, acc), W64 @ x + b + acc, rtol=1e-5, atol=1e-6)


# ---- attention ----------------------------------------------------------------------------------------------
def _rand_attn_inputs(seed, nq=4, nkv=2, T=9, max_len=16):
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal((nq + 2 * nkv) * 128).astype(F32)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(F32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(F32)
    Kc = O.bf16_round(rng.standard_normal((nkv, max_len, 128)).astype(F32))
    Vc = O.bf16_round(rng.standard_normal((nkv, max_len, 128)).astype(F32))
    rope = O.rope_table(syn.inv_freq(syn.shape("tiny")), max_len)
    return qkv, qn, kn, Kc, Vc, rope


def test_attention_single_position_returns_v():
    qkv, qn, kn, Kc, Vc, rope = _rand_attn_inputs(6)
    out = O.attention(qkv, qn, kn, 1e-6, rope, Kc, Vc, 0, 4, 2).reshape(4, 128)
    v = O.bf16_round(qkv[(4 + 2) * 128:].reshape(2, 128))
    for h in range(4):
        np.testing.assert_array_equal(out[h], v[h // 2])
    # the new K was stored rounded at position 0
    assert np.array_equal(Kc[:, 0], O.bf16_round(Kc[:, 0]))


def test_attention_uniform_keys_average_values():
    qkv, qn, kn, Kc, Vc, rope = _rand_attn_inputs(7, T=9)
    pos = 8
    k = qkv[4 * 128:6 * 128].reshape(2, 128)
    # make every prior key equal to the (normalised, rotated, rounded) new key -> all scores equal
    kk = O._rot(O._head_norm(k, kn, 1e-6), rope[pos, :64], rope[pos, 64:])
    Kc[:, :pos] = O.bf16_round(kk)[:, None, :]
    out = O.attention(qkv, qn, kn, 1e-6, rope, Kc, Vc, pos, 4, 2).reshape(4, 128)
    for h in range(4):
        np.testing.assert_allclose(out[h], Vc[h // 2, :pos + 1].mean(0), rtol=1e-5, atol=1e-6)


def _hf_layer(s, w):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer, Qwen3RotaryEmbedding

    cfg = Qwen3Config(hidden_size=s.hidden, intermediate_size=s.inter, num_attention_heads=s.nq,
                      num_key_value_heads=s.nkv, head_dim=s.head_dim, rms_norm_eps=s.eps, num_hidden_layers=1,
                      rope_parameters={"rope_type": "default", "rope_theta": s.theta}, attention_bias=False)
    cfg._attn_implementation = "eager"
    layer = Qwen3DecoderLayer(cfg, 0).float().eval()
    a, m = layer.self_attn, layer.mlp
    with torch.no_grad():
        for mod, key in ((a.q_proj, "q"), (a.k_proj, "k"), (a.v_proj, "v"), (a.o_proj, "o"), (m.gate_proj, "gate"),
                         (m.up_proj, "up"), (m.down_proj, "down"), (a.q_norm, "q_norm"), (a.k_norm, "k_norm"),
                         (layer.input_layernorm, "in_norm"), (layer.post_attention_layernorm, "post_norm")):
            mod.weight.copy_(torch.from_numpy(w[key]))
    return layer, Qwen3RotaryEmbedding(cfg)


def _oracle_layer_weights(w):
    gu = np.stack([w["gate"], w["up"]], axis=1).reshape(-1, w["gate"].shape[1])
    return {"qkv": np.concatenate([w["q"], w["k"], w["v"]]), "o": w["o"], "gu": gu, "down": w["down"],
            "in_norm": w["in_norm"], "post_norm": w["post_norm"], "qn": w["q_norm"], "kn": w["k_norm"]}


@pytest.mark.parametrize("T", [1, 5, 33])
def test_decoder_layer_matches_transformers(T):
    """f32 cache (the reference's ACT_F32 mode): the oracle layer equals transformers' Qwen3DecoderLayer
    (eager attention) fed the same prior K/V, to fp32 rounding."""
    from transformers import DynamicCache

    s = syn.shape("tiny")
    w = syn.layer_weights(11, 0, s)
    layer, rot = _hf_layer(s, w)
    rng = np.random.default_rng(12)
    pos = T - 1
    max_len = 40
    Kp = rng.standard_normal((s.nkv, max_len, 128)).astype(F32)
    Vp = rng.standard_normal((s.nkv, max_len, 128)).astype(F32)
    h = rng.standard_normal(s.hidden).astype(F32)
    rope = O.rope_table(syn.inv_freq(s), max_len)
    Kc, Vc = Kp.copy(), Vp.copy()
    ours = O.decoder_layer(h, _oracle_layer_weights(w), s.eps, rope, Kc, Vc, pos, s.nq, s.nkv, cache_bf16=False)
    cache = DynamicCache()
    if pos > 0:
        cache.update(torch.from_numpy(Kp[None, :, :pos].copy()), torch.from_numpy(Vp[None, :, :pos].copy()), 0)
    x = torch.from_numpy(h)[None, None, :]
    pid = torch.tensor([[pos]])
    with torch.no_grad():
        cos, sin = rot(x, pid)
        ref = layer(x, attention_mask=None, position_ids=pid, past_key_values=cache, use_cache=True,
                    position_embeddings=(cos, sin))[0, 0].numpy()
    err = np.max(np.abs(ours - ref)) / np.max(np.abs(ref))
    assert err < 2e-6, err
    # and the stored key/value of the new position equal transformers' cache entries
    kh, vh = cache.layers[0].keys[0, :, pos].numpy(), cache.layers[0].values[0, :, pos].numpy()
    np.testing.assert_allclose(Kc[:, pos], kh, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(Vc[:, pos], vh, rtol=1e-5, atol=1e-6)


# ---- processor and argmax -----------------------------------------------------------------------------------
def test_argmax_first_rules():
    assert O.argmax_first(np.array([1, 3, 3, 2], F32)) == 1
    assert O.argmax_first(np.array([np.nan, 1, np.nan, 1], F32)) == 1
    assert O.argmax_first(np.full(5, -np.inf, F32)) == 0
    assert O.argmax_first(np.full(5, np.nan, F32)) == 0
    assert O.argmax_first(np.array([-np.inf, -5, -np.inf], F32)) == 1


def test_process_logits_matches_torch_processor():
    rng = np.random.default_rng(13)
    V, eos = 3072, 2150
    for trial in range(50):
        lg = (rng.standard_normal(V) * 3).astype(F32)
        seen = rng.random(V) < 0.05
        sup = np.zeros(V, bool)
        sup[V - 1024:] = True
        sup[eos] = False
        ngen = trial % 4
        ours = O.process_logits(lg, seen, 1.05, sup, ngen, 2, eos)
        t = torch.from_numpy(lg)[None]
        ts = torch.from_numpy(seen)[None]
        ref = torch.where(ts, torch.where(t < 0, t * 1.05, t / 1.05), t).masked_fill(torch.from_numpy(sup)[None], -np.inf)
        if ngen < 2:
            ref[0, eos] = -np.inf
        np.testing.assert_array_equal(ours, ref[0].numpy())
        assert O.argmax_first(ours) == int(torch.argmax(ref))


# ---- code predictor composition -----------------------------------------------------------------------------
@pytest.mark.parametrize("projected", [False, True])
def test_code_predictor_frame_matches_transformers_stack(projected):
    """The code-predictor loop (inputs per position, growing cache, final norm + per-position head, greedy
    pick) against a stack of transformers' Qwen3DecoderLayer run position by position over one DynamicCache,
    Qwen3RMSNorm and a torch matmul head, f32 cache: the same codes at every position and logits to fp32
    rounding. Tiny shape, 2 layers, 6 positions. ``projected``: inputs twice as wide as the stack, each taken
    through torch.nn.functional.linear with a bias first (small_to_mtp_projection, qwen3/kernels.py:629-637)."""
    from transformers import DynamicCache
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    s = syn.shape("tiny", n_layers=2, vocab=64)
    n = 6
    rng = np.random.default_rng(21)
    layers = [syn.layer_weights(31, i, s) for i in range(s.n_layers)]
    norm = (1 + 0.1 * rng.standard_normal(s.hidden)).astype(F32)
    # large head weights so every position has a clear winner (the check is about composition, not ties)
    heads = [(0.5 * rng.standard_normal((s.vocab, s.hidden))).astype(F32) for _ in range(n - 1)]
    win = 2 * s.hidden if projected else s.hidden
    cemb = [rng.standard_normal((s.vocab, win)).astype(F32) for _ in range(n - 2)]
    temb = rng.standard_normal((96, win)).astype(F32)
    x0 = rng.standard_normal(win).astype(F32)
    id0 = 77
    rope = O.rope_table(syn.inv_freq(s), n)
    wts = {"layers": [_oracle_layer_weights(w) for w in layers], "norm": norm, "heads": heads, "cemb": cemb,
           "temb": temb, "rope": rope, "eps": s.eps, "nq": s.nq, "nkv": s.nkv}
    if projected:
        wts["proj"] = (0.05 * rng.standard_normal((s.hidden, win))).astype(F32)
        wts["proj_b"] = (0.5 * rng.standard_normal(s.hidden)).astype(F32)
    orc = O.CodePredictorOracle(wts, n, cache_bf16=False)
    codes, logits = orc.frame(x0, id0)
    hf = [_hf_layer(s, w) for w in layers]
    for i, (layer, _) in enumerate(hf):
        layer.self_attn.layer_idx = i
    fnorm = Qwen3RMSNorm(s.hidden, eps=s.eps)
    with torch.no_grad():
        fnorm.weight.copy_(torch.from_numpy(norm))
    cache = DynamicCache()
    ref_codes = [id0]
    for g in range(n):
        x = x0 if g == 0 else temb[id0] if g == 1 else cemb[g - 2][ref_codes[g - 1]]
        h = torch.from_numpy(np.asarray(x, F32))[None, None, :]
        if projected:
            h = torch.nn.functional.linear(h, torch.from_numpy(wts["proj"]), torch.from_numpy(wts["proj_b"]))
        pid = torch.tensor([[g]])
        with torch.no_grad():
            for layer, rot in hf:
                h = layer(h, attention_mask=None, position_ids=pid, past_key_values=cache, use_cache=True,
                          position_embeddings=rot(h, pid))
                h = h[0] if isinstance(h, tuple) else h
            if g == 0:
                continue
            lg = (fnorm(h)[0, 0] @ torch.from_numpy(heads[g - 1]).T).numpy()
        ref_codes.append(int(np.argmax(lg)))
        err = np.max(np.abs(logits[g - 1] - lg)) / np.max(np.abs(lg))
        assert err < 1e-5, (g, err)
    assert codes == ref_codes


# ---- batched streams ---------------------------------------------------------------------------------------
def test_bf16_terms_bounds_and_exactness():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(200000) * np.exp(rng.uniform(-20, 20, 200000))).astype(F32)
    assert np.array_equal(O.bf16_terms(x, 0), x)
    assert np.array_equal(O.bf16_terms(x, 1), O.bf16_round(x))
    # two terms keep 16 significant bits: |x - t0 - t1| <= 2^-17 |x| (two round-to-nearest steps of 2^-9 each)
    e2 = np.abs(O.bf16_terms(x, 2).astype(np.float64) - x) / np.abs(x)
    assert e2.max() <= 2.0 ** -17
    # three terms reproduce every float32 value whose exponent leaves the last term normal
    assert np.array_equal(O.bf16_terms(x, 3), x)
    # brute force on a few values: the terms are bf16 values and their fp32 sum is x
    for v in x[:50]:
        r, ts = np.float32(v), []
        for _ in range(3):
            t = np.float32(torch.tensor(float(r)).to(torch.bfloat16).float().item())
            ts.append(t)
            r = np.float32(r - t)
        assert np.float32(np.float32(ts[0] + ts[1]) + ts[2]) == v


def test_batch_oracle_rows_equal_single_stream_oracle():
    """Row b of a batched step is the M=1 talker step of stream b (same caches, same position); the head differs
    only in applying the final norm's inverse RMS after the product, so logits agree to float rounding."""
    s = syn.shape("tiny")
    rng = np.random.default_rng(2)
    layers = [syn.layer_weights(3, i, s) for i in range(s.n_layers)]
    from oracle.workload import pack_layer

    f = syn.final_weights(3, s)
    w = {"layers": [pack_layer(L, "i8row") for L in layers], "norm": f["norm"], "head": O.quantize(f["head"], "i8row")[2],
         "emb": f["emb"], "rope": O.rope_table(syn.inv_freq(s), 64), "eps": s.eps, "nq": s.nq, "nkv": s.nkv}
    B, T = 3, [5, 17, 40]
    Ks = [rng.standard_normal((s.n_layers, s.nkv, 64, 128)).astype(F32) for _ in range(B)]
    Vs = [rng.standard_normal((s.n_layers, s.nkv, 64, 128)).astype(F32) for _ in range(B)]
    Ks = [O.bf16_round(k) for k in Ks]
    Vs = [O.bf16_round(v) for v in Vs]
    tok = [7, 300, 511]
    bo = O.BatchTalkerOracle(w, [k.copy() for k in Ks], [v.copy() for v in Vs])
    lo = []
    codes, lg = bo.step(tok, T, lo)
    for b in range(B):
        so = O.TalkerOracle(w, Ks[b].copy(), Vs[b].copy())
        slo = []
        c1, lg1 = so.step(tok[b], T[b], slo)
        for i in range(s.n_layers):
            assert np.max(np.abs(lo[i][b] - slo[i])) <= 1e-5 * np.max(np.abs(slo[i]))
        assert np.max(np.abs(lg[b] - lg1)) <= 1e-5 * np.max(np.abs(lg1))
        assert codes[b] == c1
        # the step appended this stream's K/V at its own position only
        assert np.array_equal(bo.Ks[b][:, :, T[b]], so.K[:, :, T[b]])
        assert np.array_equal(bo.Ks[b][:, :, : T[b]], Ks[b][:, :, : T[b]])


def test_batch_workload_inputs_are_seeded():
    T = syn.batch_lengths(0, "batch17b")
    assert len(T) == 16 and min(T) >= 64 and max(T) <= 2048 and T == syn.batch_lengths(0, "batch17b")
    tok = syn.batch_tokens(0, "batch17b")
    assert len(tok) == 16 and max(tok) < 3072
    s = syn.workload_shape("batchsmall")
    k1, v1 = syn.batch_prefill(0, 1, 2, s, 9)
    k2, _ = syn.batch_prefill(0, 1, 3, s, 9)
    assert k1.shape == (s.nkv, 9, 128) and not np.array_equal(k1, k2)
    assert np.array_equal(O.bf16_round(k1), k1) and abs(float(v1.std()) - 1.0) < 0.05


# ---- sampled picks ------------------------------------------------------------------------------------------
PHILOX_KAT = [  # Random123 kat_vectors, philox4x32_10: counter, key, output
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


def test_philox_known_answers():
    for c, k, e in PHILOX_KAT:
        r = O.philox4x32_10(np.array(c, dtype=np.uint32), np.array(k, dtype=np.uint32))
        assert [int(x) for x in r] == list(e)
    # broadcasting over many counters gives the same words as one at a time
    ctr = np.array([[i, 7, 0, 0x51] for i in range(5)], dtype=np.uint32)
    key = np.array([3, 4], dtype=np.uint32)
    many = O.philox4x32_10(ctr, key)
    for i in range(5):
        assert np.array_equal(many[i], O.philox4x32_10(ctr[i], key))


def test_order_key_and_topk_threshold_brute_force():
    rng = np.random.default_rng(11)
    v = np.concatenate([rng.standard_normal(300).astype(F32), np.array([0.0, -0.0, 1.5, 1.5, 1.5, -np.inf], F32)])
    k = O.order_key(v)
    by_key = v[np.argsort(k, kind="stable")].astype(np.float64)
    assert np.all(np.diff(by_key) >= 0)  # keys follow the values (-0.0 sorts just below +0.0)
    assert O.order_key(np.array([-0.0], F32))[0] + 1 == O.order_key(np.array([0.0], F32))[0]
    for top_k in (1, 2, 5, 17, 100, 305, 306, 0, 400):
        thr = O.topk_threshold(v, top_k)
        if top_k <= 0 or top_k >= v.size:
            assert thr == 0
            continue
        above = int((k > thr).sum())
        at_least = int((k >= thr).sum())
        assert above < top_k <= at_least  # thr is the key of the k-th largest entry, ties included


def test_sample_draw_keep_rule():
    v = np.array([1.0, 3.0, 3.0, -np.inf, 2.0, np.nan, 0.5], F32)
    kept = set()
    for c in range(300):
        i, g = O.sample_draw(v, 1.0, 2, seed=5, counter=c)
        kept.add(i)
    # top_k = 2: the threshold is the key of 3.0, both 3.0 entries are kept; the NaN entry is never picked
    assert kept == {1, 2}
    kept = {O.sample_draw(v, 1.0, 0, 9, c)[0] for c in range(2000)}
    assert 3 not in kept and 5 not in kept and kept <= {0, 1, 2, 4, 6}
    assert O.sample_draw(np.full(4, -np.inf, F32), 1.0, 0, 1, 0)[0] == 0


def test_sample_draw_law_matches_softmax_over_top_k():
    """Gumbel-max over the kept entries is softmax sampling: the empirical frequencies of many draws (successive
    counters) match softmax(v / T) restricted to the top k within a chi-square bound."""
    from scipy.stats import chisquare

    rng = np.random.default_rng(4)
    v = (rng.standard_normal(40) * 1.5).astype(F32)
    T, top_k, n = 0.8, 12, 6000
    x = v * F32(1.0 / T)
    keep = np.argsort(-x.astype(np.float64))[:top_k]
    p = np.exp(x[keep].astype(np.float64) - float(x[keep].max()))
    p = p / p.sum()
    counts = np.zeros(v.size)
    for c in range(n):
        counts[O.sample_draw(v, 1.0 / T, top_k, seed=123, counter=c)[0]] += 1
    assert counts.sum() == counts[keep].sum()
    stat, pval = chisquare(counts[keep], p * n)
    assert pval > 1e-3, (stat, pval)
