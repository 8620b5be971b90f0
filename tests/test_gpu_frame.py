"""The persistent frame kernel (sk_talker_frames): greedy codes, logits and per-layer residuals against the oracle,
one launch for many frames against one launch per frame, graph replay, and the error word."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from sokutou_amd import synthetic as syn

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
TOL = 1e-2


def rel_err(a, b) -> float:
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else a
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def _engine(name, seed, gpu):
    eng, tok = syn.make_engine(name, seed=seed, wd="i8row", device=gpu, frame_kernel=True)
    assert eng.frame_kernel
    return eng, tok


def test_small_model_against_oracle(gpu):
    """Two 0.6B-shaped layers: 8 frames in one launch against the oracle, then per-layer residuals."""
    from oracle.workload import talker_oracle

    print("small06b: persistent kernel, 8 frames in one launch", flush=True)
    spec = syn.WORKLOADS["small06b"]
    eng, tok = _engine("small06b", 2, gpu)
    orc, otok, s = talker_oracle("small06b", 2, "i8row")
    assert otok == tok
    layer_out = []
    ref_codes, ref_logits = [], None
    t = tok
    for f in range(spec["frames"]):
        t, lg = orc.step(t, spec["kv"] + f, layer_out if f == spec["frames"] - 1 else None)
        ref_codes.append(t)
        ref_logits = lg
    eng.layer_out = torch.zeros((s.n_layers, s.hidden), device=gpu)
    eng.run_frames(spec["frames"])
    torch.cuda.synchronize()
    assert eng.frame_error() == 0, eng.frame_diag()
    codes = eng.frame_ids[: spec["frames"]].cpu().tolist()
    assert codes == ref_codes, (codes, ref_codes)
    for i in range(s.n_layers):
        assert rel_err(eng.layer_out[i], layer_out[i]) < TOL
    assert rel_err(eng.logit_t.view(-1), ref_logits) < TOL
    assert int(eng.pos.item()) == spec["kv"] + spec["frames"]
    assert int(eng.id0.item()) == ref_codes[-1] and int(eng.next_id0.item()) == ref_codes[-1]


def test_talker06b_64_frames_one_launch(gpu):
    print("talker06b: 64 frames in one launch against the oracle fixture", flush=True)
    meta = json.loads((GOLD / "talker06b_seed0.json").read_text())
    gold = np.load(GOLD / "talker06b_seed0.npz")
    eng, tok = _engine("talker06b", 0, gpu)
    assert tok == meta["start_token"]
    # frame 0 alone, with per-layer residuals
    eng.layer_out = torch.zeros((28, 1024), device=gpu)
    eng.run_frames(1)
    torch.cuda.synchronize()
    assert eng.frame_error() == 0, eng.frame_diag()
    errs = [rel_err(eng.layer_out[i], gold["layer_out0"][i]) for i in range(28)]
    print(f"per-layer max rel err {max(errs):.3e}", flush=True)
    assert max(errs) < TOL
    assert rel_err(eng.logit_t.view(-1), gold["logits_first"]) < TOL
    assert int(eng.frame_ids[0]) == meta["codes"][0]
    # the remaining 63 frames in one launch
    eng.layer_out = None
    eng.run_frames(63)
    torch.cuda.synchronize()
    assert eng.frame_error() == 0, eng.frame_diag()
    codes = [meta["codes"][0]] + eng.frame_ids[:63].cpu().tolist()
    assert codes == meta["codes"]
    assert rel_err(eng.logit_t.view(-1), gold["logits_last"]) < TOL
    assert int(eng.pos.item()) == meta["start_pos"] + 64


def test_talker06b_graph_replay_one_frame_per_launch(gpu):
    print("talker06b: captured single-frame launch replayed 64 times", flush=True)
    meta = json.loads((GOLD / "talker06b_seed0.json").read_text())
    eng, tok = _engine("talker06b", 0, gpu)
    eng.capture()
    codes = []
    for _ in range(64):
        eng.graph.replay()
        codes.append(int(eng.next_id0.item()))
    assert eng.frame_error() == 0, eng.frame_diag()
    assert codes == meta["codes"]


def test_bad_position_is_an_error_not_a_write(gpu):
    print("small06b: position beyond the cache is refused on the device", flush=True)
    eng, tok = _engine("small06b", 2, gpu)
    kc0 = eng.kc.clone()
    eng.pos.fill_(eng.max_cache)  # no room for one more frame
    eng.run_frames(1)
    torch.cuda.synchronize()
    assert eng.frame_error() == 5
    assert torch.equal(eng.kc, kc0)
    eng.frame_ws.zero_()
    eng.reset(syn.WORKLOADS["small06b"]["kv"], tok)
    eng.run_frames(2)
    torch.cuda.synchronize()
    assert eng.frame_error() == 0, eng.frame_diag()


@pytest.mark.timeout(900)
def test_talker17b_64_frames_one_launch(gpu):
    """The 1.7B shape (hidden 2048, intermediate 6144, KV 1024): per-layer residuals of frame 0, then the
    remaining 63 frames in one launch, against the oracle fixture."""
    print("talker17b: building the seeded 1.7B weights on the host (about a minute), then 64 frames", flush=True)
    meta = json.loads((GOLD / "talker17b_seed0.json").read_text())
    gold = np.load(GOLD / "talker17b_seed0.npz")
    eng, tok = _engine("talker17b", 0, gpu)
    assert tok == meta["start_token"]
    eng.layer_out = torch.zeros((28, 2048), device=gpu)
    eng.run_frames(1)
    torch.cuda.synchronize()
    assert eng.frame_error() == 0, eng.frame_diag()
    errs = [rel_err(eng.layer_out[i], gold["layer_out0"][i]) for i in range(28)]
    print(f"per-layer max rel err {max(errs):.3e}", flush=True)
    assert max(errs) < TOL
    assert rel_err(eng.logit_t.view(-1), gold["logits_first"]) < TOL
    assert int(eng.frame_ids[0]) == meta["codes"][0]
    eng.layer_out = None
    eng.run_frames(63)
    torch.cuda.synchronize()
    assert eng.frame_error() == 0, eng.frame_diag()
    codes = [meta["codes"][0]] + eng.frame_ids[:63].cpu().tolist()
    assert codes == meta["codes"]
    assert rel_err(eng.logit_t.view(-1), gold["logits_last"]) < TOL
