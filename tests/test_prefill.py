"""Prompt prefill through the talker's Hugging Face modules (Qwen3Kernels._start with ``inputs_embeds``,
qwen3/fast.py:251-263): the keys, values and last hidden state that transformers' Qwen3Model leaves for a prompt
against the oracle run position by position (CPU), then the engine's greedy frames after such a prefill against
the oracle (GPU, per-op kernels and the persistent frame kernel), and teacher forcing (teacher_logits) against
greedy generation from the same prompt."""

import numpy as np
import pytest
import torch

from oracle import talker as O
from oracle.workload import talker_oracle
from sokutou_amd import synthetic as syn

F32 = np.float32


def _oracle_prompt(name, seed, L, max_len):
    """The oracle over the prompt with fp32 weights and an fp32 cache (what an fp32 transformers model computes):
    returns (oracle, hidden state of the last position before the final norm)."""
    orc, _, s = talker_oracle(name, seed, "f32", max_len=max_len, cache_bf16=False)
    orc.K[:] = 0
    orc.V[:] = 0
    emb = syn.prompt_embeds(seed, s, L)[0]
    h = None
    for p in range(L):
        h = orc.forward(emb[p], p)
    return orc, h, s


def test_hf_prefill_cache_and_hidden_match_oracle():
    """Keys (normalised, rotated) and values of every prompt position in transformers' cache, layout
    [1, nkv, L, 128] per layer, and the last hidden state after the final norm, against the oracle."""
    from transformers import DynamicCache

    name, seed, L = "tiny", 5, 12
    s = syn.workload_shape(name)
    model = syn.hf_talker_model(seed, s)
    cache = DynamicCache()
    with torch.no_grad():
        out = model(inputs_embeds=torch.from_numpy(syn.prompt_embeds(seed, s, L)), past_key_values=cache,
                    cache_position=torch.arange(L), use_cache=True)
    orc, h, _ = _oracle_prompt(name, seed, L, max_len=40)
    assert len(cache.layers) == s.n_layers
    for i, layer in enumerate(cache.layers):
        assert tuple(layer.keys.shape) == (1, s.nkv, L, 128)
        np.testing.assert_allclose(layer.keys[0].numpy(), orc.K[i, :, :L], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(layer.values[0].numpy(), orc.V[i, :, :L], rtol=1e-4, atol=1e-6)
    ref = O.rmsnorm(h, orc.w["norm"], orc.w["eps"])
    got = out.last_hidden_state[0, -1].numpy()
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("frame_kernel", [False, True])
def test_engine_frames_after_hf_prefill(gpu, frame_kernel):
    """generate_codes with ``inputs_embeds``: the prompt through transformers' modules (fp32 weights), its keys
    and values written into the engine's bf16 cache, the first code from the codec head, then greedy frames on
    the int8 engine. The oracle: the prompt with fp32 weights and cache, its keys and values rounded to bf16,
    then the int8 oracle's greedy steps."""
    name, seed, L, frames = "small06b", 3, 24, 8
    print(f"{name}: prompt of {L} rows through transformers, then {frames} frames "
          f"({'frame kernel' if frame_kernel else 'per-op kernels'})", flush=True)
    eng, kw = syn.make_prefill_engine(name, seed, L, frames, device=gpu, frame_kernel=frame_kernel)
    assert eng.frame_kernel == frame_kernel
    codes = eng.generate_codes(kw, max_frames=frames)
    torch.cuda.synchronize()
    max_len = max(L + frames + 1, syn.WORKLOADS[name]["kv"] + 1)
    of, h, s = _oracle_prompt(name, seed, L, max_len)
    first = O.argmax_first(O.gemv(O.rmsnorm(h, of.w["norm"], of.w["eps"]), of.w["head"]))
    oi, _, _ = talker_oracle(name, seed, "i8row", max_len=max_len)
    oi.K[:] = 0
    oi.V[:] = 0
    oi.K[:, :, :L] = O.bf16_to_f32(O.bf16_bits(of.K[:, :, :L]))
    oi.V[:, :, :L] = O.bf16_to_f32(O.bf16_bits(of.V[:, :, :L]))
    # the engine's cache after the prefill holds the same bf16 keys and values
    kc = eng.kc[:, :, :L].float().cpu().numpy()
    vc = eng.vc[:, :, :L].float().cpu().numpy()
    assert np.max(np.abs(kc - oi.K[:, :, :L])) <= 1e-2 * np.max(np.abs(oi.K[:, :, :L]))
    assert np.max(np.abs(vc - oi.V[:, :, :L])) <= 1e-2 * np.max(np.abs(oi.V[:, :, :L]))
    ref = [first]
    t = first
    for f in range(frames):
        t, _ = oi.step(t, L + f)
        ref.append(t)
    assert eng.stats["prompt_tokens"] == L
    got = codes[:, 0].cpu().tolist()
    assert got == ref[: len(got)], (got, ref)
    assert len(got) == frames and int(eng.next_id0.item()) == ref[frames]
    assert int(eng.pos.item()) == L + frames


@pytest.mark.gpu
def test_teacher_logits_reproduce_greedy_frames(gpu):
    """teacher_logits (qwen3/kernels.py:714-753) fed the codes that greedy generation produced from the same
    prompt (talker with a 5-layer code predictor, 16 code groups): every talker and code-predictor logits row
    picks the code that generation chose next, on the per-op kernels against the one-launch kernels."""
    L, frames = 20, 6
    print(f"small06b + cp06b: prompt of {L} rows, {frames} greedy frames, then teacher forcing", flush=True)
    eng, kw = syn.make_prefill_engine("small06b", 4, L, frames, device=gpu, frame_kernel=True, cp="cp06b")
    assert eng.frame_kernel and eng.cpk is not None
    codes = eng.generate_codes(kw, max_frames=frames)
    nxt = int(eng.next_id0.item())
    assert codes.shape == (frames, 16)
    l0, lcp = eng.teacher_logits(kw, codes)
    assert l0.shape == (frames + 1, 3072) and lcp.shape == (frames, 15, 2048)
    assert l0.argmax(dim=1).tolist() == codes[:, 0].cpu().tolist() + [nxt]
    assert lcp.argmax(dim=2).tolist() == codes[:, 1:].cpu().tolist()
