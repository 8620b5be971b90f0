"""The stage-trace summary (sokutou_amd/stage_trace.py) on synthetic stamps, on the CPU: every step and exchange of
a layer comes out as the difference the stamps were built with, for the talker (partials and merge) and the code
predictor (whole-cache attention) layouts."""

import numpy as np
import pytest

from sokutou_amd import stage_trace as st


def _stamps(n_layers=5, step=1.0):
    """Stamps with every compute event of layer l at 100 l + offset and the control events just after them."""
    t = np.zeros((st._WG, 2, st._TRACE_LAYERS, st._TRACE_EVENTS))
    order = [st.C_S1, st.C_S1DOT, st.C_S1PUB, st.C_S2, st.C_S2END, st.C_S4, st.C_S4DOT, st.C_S4PUB, st.C_S5,
             st.C_S5DOT, st.C_S5PUB, st.C_S6, st.C_S6DOT, st.C_S6PUB]
    for l in range(n_layers):
        for k, ev in enumerate(order):
            t[:, 1, l, ev] = 100.0 * l + step * k
        base = 100.0 * l
        t[:, 0, l, st.K_S1IN] = base - 0.5                # residual ready just before S1
        t[:, 0, l, st.K_QKV] = base + step * 2 + 0.25     # q|k|v 0.25 after its publication
        t[:, 0, l, st.K_MRGPOLL] = base + step * 4 + 0.5  # partials 0.5 after the attention's end
        t[:, 0, l, st.K_ATT] = base + step * 4 + 0.75     # attention output 0.25 after the partials
        t[:, 0, l, st.K_HMID] = base + step * 7 + 0.5
        t[:, 0, l, st.K_ACT] = base + step * 10 + 0.5
    return t


def test_talker_summary():
    s = st.summarise(_stamps(), 5)
    steps = dict(s["steps"])
    assert steps["S1 qkv dot"] == 1.0 and steps["S6 publish"] == 1.0
    assert s["layer_us"] == 100.0
    ex = dict(s["exchanges"])
    assert ex["q|k|v of the head (XCD-local, 32 producers)"] == 0.25
    assert ex["attention partials (XCD-local, 32 producers)"] == 0.5
    assert ex["attention output (global, 256 producers; from the partials' arrival)"] == 0.25
    assert ex["h after o (global, 256 producers)"] == 0.5
    # every consumer is ready at the same time here, so the 90th percentile is the median
    assert dict(s["exchanges_p90"]) == pytest.approx(ex)


def test_exchange_percentile_sees_the_slow_consumers():
    """One consumer in ten of the residual exchange 1 us late: the median stays, the 90th percentile moves."""
    name = "residual h (global, 256 producers)"
    base = dict(st.summarise(_stamps(), 5)["exchanges"])[name]
    t = _stamps()
    t[::10, 0, 1:5, st.K_S1IN] += 1.0  # 26 of the 256 consumers
    s = st.summarise(t, 5)
    assert dict(s["exchanges"])[name] == pytest.approx(base)
    assert base < dict(s["exchanges_p90"])[name] <= base + 1.0


def test_code_predictor_summary_has_no_merge():
    s = st.summarise(_stamps(), 5, whole_attention=True)
    ex = dict(s["exchanges"])
    assert not any("partials" in k for k in ex)
    assert ex["attention output (global, 256 producers, written during S2)"] == 0.75
    md = st.to_markdown("cp06b", type("S", (), {"n_layers": 5, "hidden": 1024, "inter": 3072})(), s, 1000.0, 1)
    assert "positions 0 and 1 unpaired" in md and "| **layer (S1 start to next S1 start)** | **100.00** |" in md
