"""The whole 1.7B Qwen3-TTS frame on the persistent kernels: the projected code predictor (sk_cp_frame with its
2048 -> 1024 projection stage) and the 1.7B talker (sk_talker_frames fed by talker_in), one graph replay per frame,
against the whole-frame oracle fixture (frame17b: 28 talker layers, KV 1024, 8 greedy frames of 16 codes)."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from sokutou_amd import synthetic as syn

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def test_whole_17b_frame_on_the_persistent_kernels(gpu):
    meta = json.loads((GOLD / "frame17b_seed0.json").read_text())
    gold = np.load(GOLD / "frame17b_seed0.npz")
    print("frame17b: building the 1.7B talker (28 layers, KV 1024) with the projected code predictor", flush=True)
    eng, tok, kw = syn.make_frame_engine("frame17b", 0, gpu)
    assert tok == meta["start_token"]
    assert eng.frame_kernel and eng.cpk is not None and eng.cpk.proj is not None
    eng.capture()
    eng._start(kw)
    got = []
    for f in range(meta["frames"]):
        eng.graph.replay()
        got.append(eng.codes.view(-1).cpu().tolist())
        print(f"  frame {f}: {got[-1][:6]}...", flush=True)
        if f == 0:
            lg = eng.logit_t.view(-1).cpu().numpy()
            err = float(np.max(np.abs(lg - gold["logits_first"])) / np.max(np.abs(gold["logits_first"])))
            print(f"  talker logits of frame 0: max rel err {err:.2e}", flush=True)
            assert err < 1e-2
    assert eng.frame_error() == 0 and eng.cpk.error() == 0
    bad = [(f, g, got[f][g], meta["codes"][f][g]) for f in range(len(got)) for g in range(16)
           if got[f][g] != meta["codes"][f][g]]
    assert not bad, bad[:8]
