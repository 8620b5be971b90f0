"""The batched decode path (sk_tile_weights, sk_bgemm, sk_batch_frame): the M=16 GEMM against an fp32 evaluation of
the same contraction, whole steps of ragged streams against the oracle, invariance under stream order and batch
size, graph replay, and the error word."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import talker as O
from sokutou_amd import _lib
from sokutou_amd import synthetic as syn

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
TOL = 1e-2       # the bar for per-layer residuals against the fp32 oracle
TIGHT = 1e-4     # what the three-term bf16 inputs actually reach


def rel_err(a, b) -> float:
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else a
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def _terms(x: torch.Tensor) -> torch.Tensor:
    """[terms][...] bf16 planes whose fp32 sum is x."""
    n = int(_lib.load().sk_batch_terms())
    r, out = x.float().clone(), []
    for _ in range(n):
        t = r.to(torch.bfloat16)
        out.append(t)
        r = r - t.float()
    return torch.stack(out).contiguous()


def test_tile_layout(gpu):
    print("sk_tile_weights against the documented layout", flush=True)
    N, K = 48, 320
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8)
    out = torch.zeros_like(w, device=gpu)
    _lib.call("sk_tile_weights", w.to(gpu).data_ptr(), out.data_ptr(), N, K, _lib.stream())
    ref = w.view(N // 16, 16, K // 64, 4, 16).permute(0, 2, 3, 1, 4).contiguous().view(N, K)
    assert torch.equal(out.cpu(), ref)


def test_batch_attention_at_block_boundaries(gpu):
    """sk_batch_attn alone: eight streams at positions on either side of the 128-position blocks (one block, a
    block plus one position, several blocks with a one-position tail) and the cache's last row, each against the fp32
    oracle's attention over that stream's own cache; the appended K/V rows and nothing else of the caches change."""
    nkv, nq, max_len = 8, 16, 1024
    pos = [0, 63, 127, 128, 129, 255, 700, max_len - 1]
    B = len(pos)
    print(f"sk_batch_attn: {B} streams at positions {pos}", flush=True)
    rng = np.random.default_rng(11)
    width = (nq + 2 * nkv) * 128
    qkv = np.zeros((16, width), np.float32)
    qkv[:B] = rng.standard_normal((B, width)).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    Kc = O.bf16_round(rng.standard_normal((B, nkv, max_len, 128)).astype(np.float32))
    Vc = O.bf16_round(rng.standard_normal((B, nkv, max_len, 128)).astype(np.float32))
    rope = O.rope_table(syn.inv_freq(syn.shape("1.7b")), max_len)
    L = _lib.load()
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    Kg, Vg = dev(Kc).to(torch.bfloat16), dev(Vc).to(torch.bfloat16)
    nt = int(L.sk_batch_terms())
    att = torch.zeros((nt, 16, nq * 128), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(int(L.sk_batch_attn_workspace_size(nkv)), dtype=torch.uint8, device=gpu)
    posg = torch.tensor(pos, dtype=torch.int64, device=gpu)
    p = _lib.ptr
    qkvg, qng, kng, ropeg = dev(qkv), dev(qn), dev(kn), dev(rope)
    _lib.call("sk_batch_attn", p(qkvg), p(qng), p(kng), 1e-6, p(ropeg), p(Kg), p(Vg), p(posg), B, max_len, nq, nkv,
              p(att), p(ws), ws.numel(), _lib.stream())
    torch.cuda.synchronize()
    assert int(ws[:4].view(torch.int32).item()) == 0
    got = att.float().sum(0).cpu().numpy()
    Kn, Vn = Kg.float().cpu().numpy(), Vg.float().cpu().numpy()
    for b in range(B):
        Ko, Vo = Kc[b].copy(), Vc[b].copy()
        ref = O.attention(qkv[b], qn, kn, 1e-6, rope, Ko, Vo, pos[b], nq, nkv, cache_bf16=True)
        e = rel_err(got[b], ref)
        assert e < 2e-5, (b, pos[b], e)
        # the appended rows: V as given (bf16), K the same bf16 or one step away where fp32 rounding straddles a tie
        np.testing.assert_array_equal(Vn[b][:, pos[b]], Vo[:, pos[b]])
        dk = np.abs(Kn[b][:, pos[b]] - Ko[:, pos[b]])
        assert np.all(dk <= np.abs(Ko[:, pos[b]]) * 2.0 ** -7 + 1e-30)
        mask = np.ones(max_len, bool)
        mask[pos[b]] = False
        np.testing.assert_array_equal(Kn[b][:, mask], Kc[b][:, mask])
        np.testing.assert_array_equal(Vn[b][:, mask], Vc[b][:, mask])
    assert float(att[:, B:].float().abs().max()) == 0.0


@pytest.mark.parametrize("N,K", [(4096, 2048), (2048, 6144), (12288, 2048), (96, 512), (3072, 1024), (1024, 2048),
                                 (1024, 3072), (6144, 1024)])
def test_bgemm_modes_against_fp32(gpu, N, K):
    from sokutou_amd.batch import tile
    from sokutou_amd.kernels import _Lin

    print(f"sk_bgemm N={N} K={K}: modes 0/1/2 against fp32", flush=True)
    g = torch.Generator().manual_seed(N + K)
    lin = _Lin(torch.randn(N, K, generator=g) * 0.02, "i8row")
    lin.w, lin.s = lin.w.to(gpu), lin.s.to(gpu)
    wt = tile(lin)
    deq = lin.dequant().cpu().numpy()
    x = torch.randn(16, K, generator=g) * 1.7
    xp = _terms(x).to(gpu)
    npart = 5
    ssp = (torch.rand(npart, 16, generator=g) * K / npart).to(gpu)
    inv = 1.0 / np.sqrt(ssp.sum(0).cpu().numpy() / K + 1e-6)
    xv = x.numpy()
    p = _lib.ptr
    st = _lib.stream()
    ws = torch.zeros(int(_lib.load().sk_bgemm_workspace_size(N, K)), dtype=torch.uint8, device=gpu)
    # mode 0: out = (x W^T) * inv
    out = torch.zeros(16, N, device=gpu)
    _lib.call("sk_bgemm", p(xp), p(ssp), npart, 1e-6, p(wt), p(lin.s), N, K, 0, p(out), None, None, None, None, p(ws), ws.numel(), st)
    ref = (xv @ deq.T) * inv[:, None]
    e0 = rel_err(out, ref)
    # mode 1: silu(gate) * up over interleaved rows
    act = torch.zeros((xp.shape[0], 16, N // 2), dtype=torch.bfloat16, device=gpu)
    _lib.call("sk_bgemm", p(xp), p(ssp), npart, 1e-6, p(wt), p(lin.s), N, K, 1, None, p(act), None, None, None, p(ws), ws.numel(), st)
    gt, up = ref[:, 0::2], ref[:, 1::2]
    e1 = rel_err(act.float().sum(0), gt / (1 + np.exp(-gt)) * up)
    # mode 2: residual += x W^T, normalised planes of the result, per-tile sums of squares
    h0 = torch.randn(16, N, generator=g)
    h = h0.to(gpu)
    nw = (1 + 0.1 * torch.randn(N, generator=g)).to(gpu)
    xn = torch.zeros((xp.shape[0], 16, N), dtype=torch.bfloat16, device=gpu)
    sso = torch.zeros(N // 16, 16, device=gpu)
    _lib.call("sk_bgemm", p(xp), None, 0, 1e-6, p(wt), p(lin.s), N, K, 2, p(h), None, p(xn), p(nw), p(sso), p(ws), ws.numel(), st)
    href = h0.numpy() + xv @ deq.T
    e2 = rel_err(h, href)
    e3 = rel_err(xn.float().sum(0), href * nw.cpu().numpy())
    ssref = (href.reshape(16, N // 16, 16) ** 2).sum(2).T
    e4 = rel_err(sso, ssref)
    print(f"  rel errors: f32 {e0:.2e} swiglu {e1:.2e} acc {e2:.2e} norm planes {e3:.2e} sumsq {e4:.2e}", flush=True)
    assert max(e0, e1, e2, e3, e4) < 1e-5


def _run_small(gpu, name="batchsmall", seed=1, frames=None, perm=None):
    """Engine over ``name`` with the streams in order ``perm`` (default identity); returns (engine, T, tok)."""
    eng, T, tok = syn.make_batch_engine(name, seed, gpu, frames=frames)
    if perm is not None:
        eng.kc.copy_(eng.kc[:, perm].clone())
        eng.vc.copy_(eng.vc[:, perm].clone())
        T, tok = [T[i] for i in perm], [tok[i] for i in perm]
        eng.reset(T, tok)
    return eng, T, tok


def test_batchsmall_against_oracle(gpu):
    from oracle.workload import batch_oracle

    spec = syn.WORKLOADS["batchsmall"]
    F = spec["frames"]
    print(f"batchsmall: {spec['batch']} ragged streams x {F} steps against the fp32 oracle", flush=True)
    eng, T, tok = _run_small(gpu)
    orc, oT, otok, s = batch_oracle("batchsmall", 1)
    assert (oT, otok) == (T, tok)
    eng.layer_out = torch.zeros((s.n_layers, 16, s.hidden), device=gpu)
    eng.logits = torch.zeros((16, eng.V), device=gpu)
    ref_codes, t, pos = [], list(tok), list(T)
    for f in range(F):
        lo = [] if f == F - 1 else None
        t, lg = orc.step(t, pos, lo)
        ref_codes.append(t)
        pos = [p_ + 1 for p_ in pos]
    for f in range(F):
        eng.step()
    torch.cuda.synchronize()
    assert eng.error() == 0
    got = eng.picked().cpu().numpy()
    assert got.shape == (F, spec["batch"])
    assert got.tolist() == ref_codes
    errs = [rel_err(eng.layer_out[i, : spec["batch"]], lo[i]) for i in range(s.n_layers)]
    el = rel_err(eng.logits[: spec["batch"]], lg)
    print(f"  per-layer residual rel err (last step) {['%.1e' % e for e in errs]}, logits {el:.1e}", flush=True)
    assert max(errs) < TIGHT and el < TIGHT
    assert eng.pos.cpu().tolist() == [p_ + F for p_ in T]
    # rows of the unused batch slots stay zero
    assert float(eng.layer_out[:, spec["batch"]:].abs().max()) == 0.0


def test_batch_stream_order_and_batch_size_do_not_change_results(gpu):
    """Every stream's logits are bitwise the same whatever the order of the streams, and a stream alone in a
    batch of one gets the same bits as inside the batch."""
    print("batchsmall: permuted streams and a batch of one, bitwise", flush=True)
    eng, T, tok = _run_small(gpu)
    eng.logits = torch.zeros((16, eng.V), device=gpu)
    eng.step()
    eng.step()
    torch.cuda.synchronize()
    base = eng.logits[: eng.batch].clone()
    codes = eng.picked().clone()
    perm = [3, 0, 4, 1, 2]
    e2, _, _ = _run_small(gpu, perm=perm)
    e2.logits = torch.zeros((16, e2.V), device=gpu)
    e2.step()
    e2.step()
    torch.cuda.synchronize()
    assert torch.equal(e2.logits[: e2.batch], base[perm])
    assert torch.equal(e2.picked(), codes[:, perm])
    # stream 2 alone
    from sokutou_amd.batch import BatchedTalker

    s = syn.workload_shape("batchsmall")
    tts = syn.make_tts(1, s, device=gpu)
    one = BatchedTalker(tts.model.talker, 1, eng.max_len, max_frames=4, device=gpu)
    one.kc[:, 0].copy_(eng.kc[:, 2])  # the batch engine already appended 2 positions: restore the prior length
    one.vc[:, 0].copy_(eng.vc[:, 2])
    one.reset([T[2]], [tok[2]])
    one.logits = torch.zeros((16, one.V), device=gpu)
    one.step()
    one.step()
    torch.cuda.synchronize()
    assert torch.equal(one.logits[0], base[2])
    assert torch.equal(one.picked()[:, 0], codes[:, 2])


def test_batch_graph_replay_matches_eager(gpu):
    print("batchsmall: graph replay against eager steps", flush=True)
    F = syn.WORKLOADS["batchsmall"]["frames"]
    eng, T, tok = _run_small(gpu)
    for _ in range(F):
        eng.step()
    torch.cuda.synchronize()
    eager = eng.picked().clone()
    e2, _, _ = _run_small(gpu)
    e2.step()  # warm-up step, then restore the state and the appended cache position
    torch.cuda.synchronize()
    e2.capture()
    e2.kc.copy_(eng.kc)  # identical prior caches: positions >= T are rewritten by the steps below
    e2.vc.copy_(eng.vc)
    e2.reset(T, tok)
    for _ in range(F):
        e2.replay()
        torch.cuda.synchronize()  # eager work between replays, as a caller's loop has
    assert e2.error() == 0
    assert torch.equal(e2.picked(), eager)


def test_batch_error_word(gpu):
    print("batchsmall: a stream reaching the end of its cache sets the error word", flush=True)
    eng, T, tok = _run_small(gpu, frames=1)
    pos = list(T)
    pos[1] = eng.max_len - 1
    eng.reset(pos, tok)
    eng.step()
    torch.cuda.synchronize()
    assert eng.error() == 0
    eng.step()
    torch.cuda.synchronize()
    assert eng.error() == 5
    with pytest.raises(ValueError):
        eng.reset([eng.max_len] + pos[1:], tok)


def test_batch17b_against_fixture(gpu):
    """16 ragged 1.7B-shaped streams, 32 greedy steps: codes identical to the fp32 oracle, per-layer residuals of
    the first step and logits of the first and last steps within the bar."""
    meta = json.loads((GOLD / "batch17b_seed0.json").read_text())
    gold = np.load(GOLD / "batch17b_seed0.npz")
    spec = syn.WORKLOADS["batch17b"]
    F = spec["frames"]
    print(f"batch17b: 16 streams x {F} steps against the fixture", flush=True)
    eng, T, tok = syn.make_batch_engine("batch17b", 0, gpu)
    assert T == meta["lengths"] and tok == meta["tokens"]
    s = syn.workload_shape("batch17b")
    eng.layer_out = torch.zeros((s.n_layers, 16, s.hidden), device=gpu)
    eng.logits = torch.zeros((16, eng.V), device=gpu)
    eng.step()
    torch.cuda.synchronize()
    rows = meta["layer_out_streams"]
    errs = [rel_err(eng.layer_out[i, rows], gold["layer_out0"][i]) for i in range(s.n_layers)]
    e0 = rel_err(eng.logits[:16], gold["logits_first"])
    print(f"  step 0: max per-layer rel err {max(errs):.2e}, logits {e0:.2e}", flush=True)
    assert max(errs) < TOL and e0 < TOL
    for _ in range(F - 1):
        eng.step()
    torch.cuda.synchronize()
    assert eng.error() == 0
    got = eng.picked().cpu().numpy()
    ref = np.array(meta["codes"])
    print(f"  codes equal: {int((got == ref).sum())} of {ref.size}", flush=True)
    assert np.array_equal(got, ref)
    assert rel_err(eng.logits[:16], gold["logits_last"]) < TOL
