"""Talker-level parity on the GPU: one 0.6B layer against the golden single-layer fixture, the full 0.6B talker
(28 layers, KV 512) against the oracle's 64 greedy codes and per-layer residuals, and graph replay against
eager execution."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from sokutou_amd import synthetic as syn

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
TOL = 1e-2  # per-layer max relative error, max|a - b| / max|b|


def rel_err(a, b) -> float:
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else a
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def _fixture(name):
    meta = json.loads((GOLD / f"{name}.json").read_text())
    return meta, np.load(GOLD / f"{name}.npz")


def _check_inputs(meta, seed, s):
    """The generator still produces the fixture's inputs (catches drift of numpy or the seeding scheme)."""
    w = syn.layer_weights(seed, 0, s)
    for k, v in w.items():
        key = f"layer0.{k}" if "all_layers" in meta["digests"] else k
        assert syn.sha256(v) == meta["digests"][key], k


def test_single_layer_06b(gpu):
    print("layer06b: 0.6B layer, pos 256", flush=True)
    meta, gold = _fixture("layer06b_seed0")
    s = syn.workload_shape("layer06b")
    _check_inputs(meta, 0, s)
    eng, _ = syn.make_engine("layer06b", seed=0, wd="i8row", device=gpu, frames=1)
    h = torch.from_numpy(gold["h"]).to(gpu)
    eng.ht.copy_(h)
    eng.pos.fill_(meta["pos"])
    with torch.no_grad():
        P = eng.T
        eng._layers(P, eng.ht, eng.qkv_t, eng.att_t, eng.act_t, eng.tk, eng.tv, eng.pos, 0)
    torch.cuda.synchronize()
    err = rel_err(eng.ht, gold["out"])
    print(f"layer06b max rel err {err:.3e}", flush=True)
    assert err < TOL
    assert err < 1e-5  # fp32 accumulation: far inside the tolerance
    kn = eng.kc[0, :, meta["pos"]].float().cpu().numpy()
    vn = eng.vc[0, :, meta["pos"]].float().cpu().numpy()
    assert np.mean(kn != gold["k_new"]) < 0.02
    np.testing.assert_array_equal(vn, gold["v_new"])


@pytest.mark.parametrize("name,seed", [("tiny", 1), ("talker06b", 0)])
def test_greedy_frames_match_oracle(gpu, name, seed):
    print(f"{name}: greedy frames against the oracle fixture", flush=True)
    meta, gold = _fixture(f"{name}_seed{seed}")
    s = syn.workload_shape(name)
    _check_inputs(meta, seed, s)
    eng, tok = syn.make_engine(name, seed=seed, wd=meta["wd"], device=gpu)
    assert tok == meta["start_token"]
    # frame 0 eagerly, layer by layer
    trace = eng.layer_trace(tok, meta["start_pos"])
    errs = [rel_err(trace[i], gold["layer_out0"][i]) for i in range(s.n_layers)]
    print(f"{name} per-layer max rel err: max {max(errs):.3e}", flush=True)
    assert max(errs) < TOL
    assert rel_err(trace[-1].view(-1), gold["logits_first"]) < TOL
    # all frames through the captured graph
    eng.reset(meta["start_pos"], tok)
    eng.capture()
    codes = []
    for _ in range(meta["frames"]):
        eng.graph.replay()
        codes.append(int(eng.next_id0.item()))
    assert codes == meta["codes"], (codes, meta["codes"])
    assert int(eng.pos.item()) == meta["start_pos"] + meta["frames"]
    assert rel_err(eng.logit_t.view(-1), gold["logits_last"]) < TOL


def test_graph_replay_equals_eager(gpu):
    print("tiny: graph replay vs eager", flush=True)
    eng, tok = syn.make_engine("tiny", seed=3, device=gpu)
    pos0 = syn.WORKLOADS["tiny"]["kv"]
    kc0, vc0 = eng.kc.clone(), eng.vc.clone()
    eager = []
    for _ in range(6):
        eng._frame()
        eager.append((int(eng.next_id0.item()), eng.logit_t.clone()))
    eng.kc.copy_(kc0)
    eng.vc.copy_(vc0)
    eng.reset(pos0, tok)
    eng.capture()
    for i in range(6):
        eng.graph.replay()
        torch.cuda.synchronize()
        assert int(eng.next_id0.item()) == eager[i][0]
        assert torch.equal(eng.logit_t, eager[i][1])


def test_generate_codes_loop(gpu):
    """The host frame loop (qwen3/fast.py:221-249 semantics): stops at the frame cap, counts cache limits."""
    eng, tok = syn.make_engine("tiny", seed=1, device=gpu)
    eng.capture()
    from sokutou_amd.fast import Sampling

    kw = {"prefill_len": syn.WORKLOADS["tiny"]["kv"], "first_token": tok, "do_sample": False, "subtalker_dosample": False,
          "repetition_penalty": 1.0, "min_new_tokens": 0}
    assert Sampling.from_kwargs(kw) == eng.s
    codes = eng.generate_codes(kw, max_frames=5)
    meta = json.loads((GOLD / "tiny_seed1.json").read_text())
    assert codes.shape == (5, 1)
    assert codes[:, 0].tolist() == [tok] + meta["codes"][:4]
    assert eng.stats["frame_limited"] and not eng.stats["stopped"]
    with pytest.raises(ValueError):
        eng.generate_codes(dict(kw, top_p=0.5))


def test_sampled_generation_matches_oracle(gpu):
    """do_sample with the talker processor through the fused sampler (qwen3/kernels.py:676-693, 709-713): the key
    comes from torch's CPU generator, the counter is the frame index; every code equals the oracle's draw."""
    from oracle import talker as O
    from oracle.workload import talker_oracle
    from sokutou_amd.fast import Sampling

    smp = Sampling(do_sample=True, temperature=0.9, top_k=50, repetition_penalty=1.05, min_new_tokens=2,
                   max_new_tokens=64)
    name, seed = "tiny", 2
    eng, tok = syn.make_engine(name, seed=seed, device=gpu, sampling=smp, suppress_tail=64, max_cache=60)
    pos0 = syn.WORKLOADS[name]["kv"]
    eng.capture()
    kw = {"prefill_len": pos0, "first_token": tok, "do_sample": True, "temperature": 0.9, "top_k": 50,
          "repetition_penalty": 1.05, "min_new_tokens": 2, "max_new_tokens": 64, "subtalker_dosample": True}
    torch.manual_seed(1234)
    codes = eng.generate_codes(kw, max_frames=20)[:, 0].tolist()
    torch.manual_seed(1234)
    key = int(torch.randint(0, 2**62, (1,)).item())
    orc, otok, s = talker_oracle(name, seed, "i8row", max_len=60)
    assert otok == tok
    V, eos = s.vocab, eng.eos
    sup = np.zeros(V, bool)
    sup[V - 64:] = True
    sup[eos] = False
    seen = np.zeros(V, bool)
    seen[tok] = True
    ngen, t, ref = 1, tok, []
    for f in range(20):
        if t == eos:
            break
        ref.append(t)
        lg = orc.logits(orc.forward(orc.w["emb"][t], pos0 + f))
        v = O.process_logits(lg, seen, 1.05, sup, ngen, 2, eos)
        t, _ = O.sample_draw(v, float(np.float32(1.0 / 0.9)), 50, key, f)
        seen[t] = True
        ngen += 1
    print(f"sampled tiny: {len(codes)} frames, {len(set(codes))} distinct codes", flush=True)
    assert codes == ref
    assert len(set(codes)) > 3


def _full_frame_oracle(seed, frames, sub_sample=None, sample=None, key=0, wd="i8row"):
    """Talker (2 layers of the 0.6B shape) + code predictor (5 layers, 2048-way heads) + talker_in, composed as the
    reference's frame (qwen3/kernels.py:666-693): code predictor from (ph32, code 0), then the talker on the sum of
    the 16 code embeddings plus the pad row. Picks greedy unless (temperature, top_k) are given for the sub-codes
    / code 0; sampled picks share one draw counter in frame order, as the one fused sampler does."""
    from oracle import talker as O
    from oracle.workload import cp_oracle, talker_oracle

    torc, tok, s = talker_oracle("small06b", seed, wd, max_len=80)
    corc, cs = cp_oracle("cp06b", seed, wd=wd)
    temb = torc.w["emb"]
    corc.w["temb"] = temb
    w = syn.cp_weights(seed, cs, 16, talker_vocab=s.vocab)
    tabs = [temb] + [O.bf16_round(t) for t in w["cemb"]] + [np.zeros_like(temb[:2048])]
    pad = syn.bf16_values(syn.normal(seed, syn.CP_FRAME0 - 1, "emb", (s.hidden,), 0.02))
    ph32, _ = syn.cp_frame_inputs(seed, 0, s)
    pos, t, cnt, out = syn.WORKLOADS["small06b"]["kv"], tok, 0, []
    for f in range(frames):
        if sub_sample is None:
            codes = corc.frame(ph32, t)[0]
        else:
            codes = [t]
            K = np.zeros((5, 8, 16, 128), np.float32)
            V = np.zeros_like(K)
            for g in range(16):
                x = ph32 if g == 0 else (temb[codes[0]] if g == 1 else corc.w["cemb"][g - 2][codes[g - 1]])
                h = np.asarray(x, np.float32)
                for i, L in enumerate(corc.w["layers"]):
                    h = O.decoder_layer(h, L, cs.eps, corc.w["rope"], K[i], V[i], g, cs.nq, cs.nkv)
                if g == 0:
                    continue
                lg = O.rms_gemv(h, corc.w["norm"], cs.eps, corc.w["heads"][g - 1])
                codes.append(O.sample_draw(lg, float(np.float32(1.0 / sub_sample[0])), sub_sample[1], key, cnt)[0])
                cnt += 1
        out.append(list(codes))
        x = np.zeros(s.hidden, np.float32)
        for g in range(16):
            x = x + tabs[g][codes[g]]
        x = x + pad
        h = torc.forward(x, pos + f)
        ph32 = O.rmsnorm(h, torc.w["norm"], s.eps)
        lg = O.gemv(ph32, torc.w["head"])
        if sample is None:
            t = O.argmax_first(lg)
        else:
            t = O.sample_draw(lg, float(np.float32(1.0 / sample[0])), sample[1], key, cnt)[0]
            cnt += 1
    return out, tok, pad


@pytest.mark.parametrize("mode", ["greedy", "greedy_frame_kernel", "sampled_per_op", "sampled",
                                  "sampled_frame_kernel", "greedy_frame_kernel_i8g32", "greedy_frame_kernel_bf16"])
def test_full_frame_with_code_predictor_matches_oracle(gpu, mode):
    """The reference's whole frame: 15 sub-codes from the code predictor (one launch, greedy or with the fused
    sampler's draws inside it; ``sampled_per_op`` runs its positions on the per-op kernels and the fused sampler),
    then the talker on talker_in of all 16 codes (per-op kernels, or one launch of the persistent talker kernel fed
    by talker_in, greedy or sampled). The one draw counter runs through sub-codes and code 0 in frame order.
    ``greedy_frame_kernel_i8g32`` / ``_bf16``: the reference's serving format and its Qwen3Kernels default, every
    kernel of the frame persistent."""
    from sokutou_amd.fast import Sampling
    from sokutou_amd.kernels import Qwen3Kernels

    seed, F = 4, 6
    s = syn.workload_shape("small06b")
    cs = syn.workload_shape("cp06b")
    tts, pad = syn.make_tts_with_cp(seed, s, cs, device=gpu)
    if mode.startswith("greedy"):
        smp = Sampling.greedy(processor=False, max_new_tokens=64)
    else:
        smp = Sampling(do_sample=True, temperature=0.9, top_k=50, repetition_penalty=1.0, min_new_tokens=0,
                       max_new_tokens=64, sub_do_sample=True, sub_temperature=0.8, sub_top_k=40)
    wd = mode.rsplit("_", 1)[1] if mode.endswith(("i8g32", "bf16")) else "i8row"
    eng = Qwen3Kernels(tts, smp, max_cache=80, wd=wd, sampler="fused", suppress_tail=0,
                       frame_kernel="frame_kernel" in mode)
    assert eng.cpk is not None
    assert ("frame_kernel" in mode) == eng.frame_kernel
    if mode == "sampled_per_op":
        eng.cpk = None  # the code predictor's positions on the per-op kernels
    kv = syn.WORKLOADS["small06b"]["kv"]
    for i in range(s.n_layers):
        k, v = syn.kv_prefill(seed, i, s, kv)
        eng.kc[i, :, :kv].copy_(torch.from_numpy(k).to(eng.kc.dtype))
        eng.vc[i, :, :kv].copy_(torch.from_numpy(v).to(eng.vc.dtype))
    tok = syn.start_token(seed, s)
    ph32, _ = syn.cp_frame_inputs(seed, 0, s)
    eng.reset(kv, tok)  # capture's warm-up frames write the cache at the current position: keep them past the prefill
    eng.capture()
    kw = {"prefill_len": kv, "first_token": tok, "last_hidden": torch.from_numpy(ph32), "tts_pad_embed": torch.from_numpy(pad),
          "do_sample": smp.do_sample, "temperature": smp.temperature, "top_k": smp.top_k,
          "repetition_penalty": smp.repetition_penalty, "min_new_tokens": smp.min_new_tokens, "max_new_tokens": 64,
          "subtalker_dosample": smp.sub_do_sample, "subtalker_temperature": smp.sub_temperature,
          "subtalker_top_k": smp.sub_top_k}
    torch.manual_seed(77)
    got = eng.generate_codes(kw, max_frames=F).cpu().tolist()
    torch.manual_seed(77)
    key = int(torch.randint(0, 2**62, (1,)).item())
    print(f"full frame ({mode}): building the oracle", flush=True)
    if mode.startswith("greedy"):
        ref, otok, _ = _full_frame_oracle(seed, F, wd=wd)
    else:
        ref, otok, _ = _full_frame_oracle(seed, F, sub_sample=(0.8, 40), sample=(0.9, 50), key=key)
    assert otok == tok
    print(f"full frame ({mode}): {len(got)} frames x 16 codes; first {got[0][:6]}", flush=True)
    bad = [(f, g, got[f][g], ref[f][g]) for f in range(len(got)) for g in range(16) if got[f][g] != ref[f][g]]
    if bad:
        print(f"  first mismatches (frame, group, gpu, oracle): {bad[:6]}", flush=True)
    # the loop stops early only if code 0 is EOS (possible when sampling)
    assert got == ref[: len(got)] and (len(got) == F or ref[len(got)][0] == eng.eos)
