"""Builds the oracle for a named synthetic workload (TEST INFRASTRUCTURE ONLY, see oracle/__init__.py).

The weights, prior cache and start token come from ``sokutou_amd.synthetic`` (the shared seeded input
generator); quantisation, packing and all arithmetic are the oracle's own (oracle/talker.py), so the GPU path
and the oracle meet only at the raw fp32 inputs.
"""

from __future__ import annotations

import hashlib

import numpy as np

from sokutou_amd import synthetic as syn

from . import talker as O


def pack_layer(w: dict, wd: str) -> dict:
    """q/k/v rows concatenated, gate/up rows interleaved (row 2n gate n, 2n+1 up n) as the reference's _Stack
    does (qwen3/kernels.py:462-469), each quantised with the oracle's quantiser and dequantised to fp32."""
    gu = np.stack([w["gate"], w["up"]], axis=1).reshape(-1, w["gate"].shape[1])
    return {"qkv": O.quantize(np.concatenate([w["q"], w["k"], w["v"]]), wd)[2], "o": O.quantize(w["o"], wd)[2],
            "gu": O.quantize(gu, wd)[2], "down": O.quantize(w["down"], wd)[2], "in_norm": w["in_norm"],
            "post_norm": w["post_norm"], "qn": w["q_norm"], "kn": w["k_norm"]}


def talker_oracle(name: str, seed: int = 0, wd: str = "i8row", max_len: int | None = None,
                  cache_bf16: bool = True, digests: dict | None = None):
    """Returns (TalkerOracle, start token, shape) for ``name`` with the prior cache loaded.
    When ``digests`` is a dict it receives SHA-256 digests of the generated inputs."""
    spec = syn.WORKLOADS[name]
    s = syn.workload_shape(name)
    T = spec["kv"]
    max_len = max_len or (T + spec.get("frames", 1) + 1)
    layers = []
    K = np.zeros((s.n_layers, s.nkv, max_len, 128), np.float32)
    V = np.zeros_like(K)
    all_h = hashlib.sha256()
    for i in range(s.n_layers):
        w = syn.layer_weights(seed, i, s)
        for k in sorted(w):
            d = syn.sha256(w[k])
            all_h.update(d.encode())
            if digests is not None and i == 0:
                digests[f"layer0.{k}"] = d
        layers.append(pack_layer(w, wd))
        k, v = syn.kv_prefill(seed, i, s, T)
        K[i, :, :T] = k
        V[i, :, :T] = v
        if digests is not None and i == 0:
            digests["layer0.kcache"] = syn.sha256(k)
            digests["layer0.vcache"] = syn.sha256(v)
    f = syn.final_weights(seed, s)
    if digests is not None:
        digests["all_layers"] = all_h.hexdigest()
        for k in sorted(f):
            digests[f"final.{k}"] = syn.sha256(f[k])
    weights = {"layers": layers, "norm": f["norm"], "head": O.quantize(f["head"], wd)[2], "emb": f["emb"],
               "rope": O.rope_table(syn.inv_freq(s), max_len), "eps": s.eps, "nq": s.nq, "nkv": s.nkv}
    return O.TalkerOracle(weights, K, V, cache_bf16), syn.start_token(seed, s), s


def cp_oracle(name: str = "cp06b", seed: int = 0, wd: str = "i8row", cache_bf16: bool = True,
              digests: dict | None = None, positions: int | None = None):
    """Returns (CodePredictorOracle, shape) for a code-predictor workload, weights quantised by the oracle;
    ``positions`` overrides the workload's count of positions (and so of heads and code tables)."""
    spec = syn.WORKLOADS[name]
    s = syn.workload_shape(name)
    n = positions or spec["positions"]
    w = syn.cp_weights(seed, s, n, in_hidden=spec.get("in_hidden"))
    if digests is not None:
        digests["layer0.q"] = syn.sha256(w["layers"][0]["q"])
        digests["head1"] = syn.sha256(w["heads"][0])
        digests["cemb2"] = syn.sha256(w["cemb"][0])
        digests["temb"] = syn.sha256(w["temb"])
    weights = {"layers": [pack_layer(L, wd) for L in w["layers"]], "norm": w["norm"],
               "heads": [O.quantize(h, wd)[2] for h in w["heads"]], "cemb": w["cemb"], "temb": w["temb"],
               "rope": O.rope_table(syn.inv_freq(s), n), "eps": s.eps, "nq": s.nq, "nkv": s.nkv}
    if "proj" in w:  # a projected code predictor: its input projection, quantised as the layers are
        weights["proj"] = O.quantize(w["proj"], wd)[2]
        weights["proj_b"] = w["proj_b"]
        if digests is not None:
            digests["proj"] = syn.sha256(w["proj"])
    return O.CodePredictorOracle(weights, n, cache_bf16), s


def batch_oracle(name: str, seed: int = 0, frames: int | None = None, cache_bf16: bool = True, act_terms: int = 0,
                 streams: list | None = None):
    """Returns (BatchTalkerOracle, lengths, tokens, shape) for a batched workload: the talker's weights quantised
    by the oracle, every stream's prior cache regenerated. ``streams`` selects a subset of the streams."""
    spec = syn.WORKLOADS[name]
    s = syn.workload_shape(name)
    frames = spec["frames"] if frames is None else frames
    T = syn.batch_lengths(seed, name)
    tok = syn.batch_tokens(seed, name)
    streams = list(range(spec["batch"])) if streams is None else list(streams)
    layers = [pack_layer(syn.layer_weights(seed, i, s), "i8row") for i in range(s.n_layers)]
    f = syn.final_weights(seed, s)
    max_len = syn.batch_max_len(name, frames)
    weights = {"layers": layers, "norm": f["norm"], "head": O.quantize(f["head"], "i8row")[2], "emb": f["emb"],
               "rope": O.rope_table(syn.inv_freq(s), max_len), "eps": s.eps, "nq": s.nq, "nkv": s.nkv}
    Ks, Vs = [], []
    for b in streams:
        n = T[b] + frames + 1
        K = np.zeros((s.n_layers, s.nkv, n, 128), np.float32)
        V = np.zeros_like(K)
        for i in range(s.n_layers):
            k, v = syn.batch_prefill(seed, i, b, s, T[b])
            K[i, :, :T[b]] = k
            V[i, :, :T[b]] = v
        Ks.append(K)
        Vs.append(V)
    orc = O.BatchTalkerOracle(weights, Ks, Vs, cache_bf16, act_terms)
    return orc, [T[b] for b in streams], [tok[b] for b in streams], s


def frame_oracle(name: str, seed: int = 0, wd: str = "i8row", frames: int | None = None, detail: bool = False):
    """Greedy whole Qwen3-TTS frames of a frame workload (the composition of the reference's ``_frame``,
    qwen3/kernels.py:666-693): the code predictor from (ph32, code 0) gives sub-codes 1..15, then the talker runs on
    talker_in, the sum of the 16 codes' embedding rows in group order (code 0 from the talker's table, code g from
    code table g - 1) plus the pad row, and its final norm's output is the next frame's ph32. ph32 starts as the
    synthetic last hidden state (``cp_frame_inputs`` at the talker's width), code 0 as the start token. Returns
    (codes [frames][16], start token) or, with ``detail``, also the top-1/top-2 margins of every pick per frame
    and the talker's logits per frame."""
    spec = syn.WORKLOADS[name]
    frames = spec["frames"] if frames is None else frames
    cspec = syn.WORKLOADS[spec["cp"]]
    torc, tok, s = talker_oracle(name, seed, wd, max_len=spec["kv"] + frames + 1)
    corc, cs = cp_oracle(spec["cp"], seed, wd=wd)
    G = cspec["positions"]
    temb = torc.w["emb"]
    corc.w["temb"] = temb
    w = syn.cp_weights(seed, cs, G, talker_vocab=s.vocab, in_hidden=cspec.get("in_hidden"))
    tabs = [temb] + [O.bf16_round(t) for t in w["cemb"]] + [np.zeros_like(temb)]
    pad = syn.bf16_values(syn.normal(seed, syn.CP_FRAME0 - 1, "emb", (s.hidden,), 0.02))
    ph32, _ = syn.cp_frame_inputs(seed, 0, s)
    pos, t, out, margins, logits = spec["kv"], tok, [], [], []
    for f in range(frames):
        codes, clg = corc.frame(ph32, t)
        out.append([int(c) for c in codes])
        x = np.zeros(s.hidden, np.float32)
        for g in range(G):
            x = x + tabs[g][codes[g]]
        x = x + pad
        h = torc.forward(x, pos + f)
        ph32 = O.rmsnorm(h, torc.w["norm"], s.eps)
        lg = O.gemv(ph32, torc.w["head"])
        t = O.argmax_first(lg)
        margins.append([float(np.diff(np.sort(v)[-2:])[0]) for v in (*clg, lg)])
        logits.append(lg)
    return (out, tok, margins, logits) if detail else (out, tok)

