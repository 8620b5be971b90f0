"""Per-stage timing of the persistent frame kernel from its own trace stamps.

    python -m sokutou_amd.stage_trace [talker06b|talker17b|cp06b] [--frames N]

The kernel keeps optional wall-clock stamps (100 MHz) of frame 0 of a launch for every workgroup and layer when
the workspace's trace word is set: the compute waves stamp the start of each stage (after its barrier), the end of
each dot and their publication; the control wave stamps when each stage's input has arrived and been staged. This
tool runs one traced launch of the synthetic workload (for the code predictor: one frame with positions 0 and 1
unpaired, so that frame 0 of the launch is position 0's pass), then prints, as markdown:

* the median time of each step of a layer (median over the 256 workgroups and the middle layers);
* each exchange: from the last producer's publication to a consumer's input being ready (the median, and the 90th
  percentile over every consumer and layer);
* the median layer time.

This is the reference's per-frame profiling role (qwen3/prof_frame.py:41-87, which times the frame's kernels with
CUDA events) for a kernel that runs a whole frame in one launch.
"""

from __future__ import annotations

import argparse
import sys

import numpy as np
import torch

from . import synthetic as syn

# trace layout: [workgroup 256][role 2: control, compute][layer 32][event 16] of int64 stamps, from byte 256 of the
# workspace (after its control words)
_TRACE_LAYERS, _TRACE_EVENTS, _WG, _TRACE_AT = 32, 16, 256, 256
# compute-wave events
C_S1, C_S1DOT, C_S1PUB, C_S2, C_S2END, C_S4, C_S4DOT, C_S4PUB = 0, 8, 1, 2, 3, 4, 9, 5
C_S5, C_S5DOT, C_S5PUB, C_S6, C_S6DOT, C_S6PUB = 12, 10, 6, 13, 11, 7
# control-wave events
K_START, K_S1IN, K_QKV, K_ATTB, K_MRGPOLL, K_MRGDONE, K_ATT, K_HMID, K_ACT = 0, 1, 2, 3, 8, 4, 5, 6, 7


def traced_launch(name: str, frames: int = 2):
    """Builds the workload's engine, warms it up, then runs one launch of ``frames`` frames (the code predictor:
    one frame of all its positions) with tracing on. Returns (stamps in us as float64 [256, 2, 32, 16], shape, us
    of the launch)."""
    dev = torch.device("cuda:0")
    s = syn.workload_shape(name)
    nbytes = _WG * 2 * _TRACE_LAYERS * _TRACE_EVENTS * 8
    if name == "cp06b":
        eng = syn.make_cp_engine(name, 0, dev, keep_layers=True, pair=False)
        x0, id0 = syn.cp_frame_inputs(0, 0, s)
        eng.x0.copy_(torch.from_numpy(x0))
        eng.id0.fill_(id0)
        ws, run, err = eng.ws, eng.run, eng.error
    else:
        eng, tok = syn.make_engine(name, seed=0, wd="i8row", device=dev, frame_kernel=True)
        kv = syn.WORKLOADS[name]["kv"]
        ws, err = eng.frame_ws, eng.frame_error

        def run():
            eng.reset(kv, tok)
            eng.run_frames(frames)
    for _ in range(3):
        run()
    ws[32:36].view(torch.int32).fill_(1)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    run()
    e1.record()
    torch.cuda.synchronize()
    if err():
        raise RuntimeError(f"frame kernel error {err()}")
    raw = ws[_TRACE_AT:_TRACE_AT + nbytes].view(torch.int64).view(_WG, 2, _TRACE_LAYERS, _TRACE_EVENTS)
    ws[32:36].zero_()
    return raw.cpu().numpy().astype(np.float64) * 0.01, s, e0.elapsed_time(e1) * 1e3


def summarise(t: np.ndarray, n_layers: int, whole_attention: bool = False) -> dict:
    """Medians of the layer steps and exchanges over workgroups and the middle layers (1 .. n_layers - 2).
    ``whole_attention``: every workgroup attends over the whole cache (the code predictor), so there are no
    partials to merge and the attention output is written by the workgroups themselves during S2."""
    ctl, cmp_ = t[:, 0], t[:, 1]
    layers = range(1, min(n_layers, _TRACE_LAYERS) - 1)
    xcd = np.arange(_WG) // 32  # the kernel's dense rank: workgroup g = 32 * XCD + rank

    def med(f):
        return float(np.median([f(l) for l in layers]))

    steps = [
        ("S1 qkv dot", lambda l: np.median(cmp_[:, l, C_S1DOT] - cmp_[:, l, C_S1])),
        ("S1 publish", lambda l: np.median(cmp_[:, l, C_S1PUB] - cmp_[:, l, C_S1DOT])),
        ("S1 publish -> S2 start (qkv exchange, XCD-local)", lambda l: np.median(cmp_[:, l, C_S2] - cmp_[:, l, C_S1PUB])),
        ("S2 attention (norm, RoPE, scores, softmax, PV, partial published)", lambda l: np.median(cmp_[:, l, C_S2END] - cmp_[:, l, C_S2])),
        ("S2 end -> S4 start (partials exchange, merge, attention-output exchange)", lambda l: np.median(cmp_[:, l, C_S4] - cmp_[:, l, C_S2END])),
        ("S4 o dot", lambda l: np.median(cmp_[:, l, C_S4DOT] - cmp_[:, l, C_S4])),
        ("S4 publish", lambda l: np.median(cmp_[:, l, C_S4PUB] - cmp_[:, l, C_S4DOT])),
        ("S4 publish -> S5 start (h after o exchange, RMSNorm staging)", lambda l: np.median(cmp_[:, l, C_S5] - cmp_[:, l, C_S4PUB])),
        ("S5 gate/up dot", lambda l: np.median(cmp_[:, l, C_S5DOT] - cmp_[:, l, C_S5])),
        ("S5 SwiGLU + publish", lambda l: np.median(cmp_[:, l, C_S5PUB] - cmp_[:, l, C_S5DOT])),
        ("S5 publish -> S6 start (activation exchange)", lambda l: np.median(cmp_[:, l, C_S6] - cmp_[:, l, C_S5PUB])),
        ("S6 down dot", lambda l: np.median(cmp_[:, l, C_S6DOT] - cmp_[:, l, C_S6])),
        ("S6 publish", lambda l: np.median(cmp_[:, l, C_S6PUB] - cmp_[:, l, C_S6DOT])),
        ("S6 publish -> next S1 start (residual exchange, RMSNorm staging)", lambda l: np.median(cmp_[:, l + 1, C_S1] - cmp_[:, l, C_S6PUB])),
    ]

    def local_last(l, ev):  # per consumer: the last publication among the 32 workgroups of its XCD
        last = np.array([cmp_[xcd == x, l, ev].max() for x in range(8)])
        return last[xcd]

    # per consumer workgroup: its input ready, less the last producer's publication
    if whole_attention:
        att = [("attention output (global, 256 producers, written during S2)",
                lambda l: ctl[:, l, K_ATT] - cmp_[:, l, C_S2END].max())]
    else:
        att = [("attention partials (XCD-local, 32 producers)", lambda l: ctl[:, l, K_MRGPOLL] - local_last(l, C_S2END)),
               ("attention output (global, 256 producers; from the partials' arrival)",
                lambda l: ctl[:, l, K_ATT] - ctl[:, l, K_MRGPOLL])]
    exchanges = [
        ("residual h (global, 256 producers)", lambda l: ctl[:, l + 1, K_S1IN] - cmp_[:, l, C_S6PUB].max()),
        ("q|k|v of the head (XCD-local, 32 producers)", lambda l: ctl[:, l, K_QKV] - local_last(l, C_S1PUB)),
        *att,
        ("h after o (global, 256 producers)", lambda l: ctl[:, l, K_HMID] - cmp_[:, l, C_S4PUB].max()),
        ("SwiGLU activation (global, 256 producers)", lambda l: ctl[:, l, K_ACT] - cmp_[:, l, C_S5PUB].max()),
    ]

    def p90(f):  # over every consumer and layer
        return float(np.percentile(np.concatenate([f(l) for l in layers]), 90))

    layer = med(lambda l: np.median(cmp_[:, l + 1, C_S1] - cmp_[:, l, C_S1]))
    return {"steps": [(n, med(f)) for n, f in steps],
            "exchanges": [(n, med(lambda l, f=f: np.median(f(l)))) for n, f in exchanges],
            "exchanges_p90": [(n, p90(f)) for n, f in exchanges],
            "layer_us": layer, "layers": f"{layers.start}..{layers.stop - 1}"}


def to_markdown(name: str, s, summ: dict, launch_us: float, frames: int) -> str:
    what = ("one traced launch of one frame, positions 0 and 1 unpaired ({:.1f} us, stamps of position 0)".format(launch_us)
            if name == "cp06b" else f"one traced launch of {frames} frames ({launch_us:.1f} us, stamps of frame 0)")
    out = [f"Workload {name}: {s.n_layers} layers, hidden {s.hidden}, intermediate {s.inter}; {what}. Medians over "
           f"the 256 workgroups and layers {summ['layers']}.", "", "| step of a layer | us |", "|---|---|"]
    out += [f"| {n} | {v:.2f} |" for n, v in summ["steps"]]
    out += [f"| **layer (S1 start to next S1 start)** | **{summ['layer_us']:.2f}** |", "",
            "| exchange: last producer's publication -> consumer's input ready | median us | p90 us |", "|---|---|---|"]
    out += [f"| {n} | {v:.2f} | {q:.2f} |" for (n, v), (_, q) in zip(summ["exchanges"], summ["exchanges_p90"])]
    return "\n".join(out)


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("workload", nargs="?", default="talker06b", choices=["talker06b", "talker17b", "cp06b"])
    ap.add_argument("--frames", type=int, default=2)
    a = ap.parse_args(argv)
    t, s, us = traced_launch(a.workload, a.frames)
    print(to_markdown(a.workload, s, summarise(t, s.n_layers, a.workload == "cp06b"), us, a.frames), flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
