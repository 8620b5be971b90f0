"""The real-model surface of the engine on the CPU (no kernels launched): prompt interception from the official
``generate_custom_voice`` (qwen3/fast.py:127-147), the engine's KV cache shared with the talker's Hugging Face
modules (``tcache``, qwen3/fast.py:91-92, qwen3/kernels.py:695-703), the eager speech-tokenizer decode, and every
engine attribute the reference's callers use (qwen3/serve.py, bench.py, check.py, prof_frame.py)."""

import inspect
import re

import numpy as np
import pytest
import torch

from sokutou_amd import synthetic as syn
from sokutou_amd.fast import Qwen3Fast, Sampling


def test_prompt_intercepts_generate_and_restores_it():
    tts = syn.make_hf_tts("tiny", seed=3)
    talker = tts.model.talker
    original = talker.generate
    probe = Qwen3Fast(tts, graphs=False)
    kw = probe.prompt("hello there", "vivian", "english")
    s = syn.workload_shape("tiny")
    assert tuple(kw["inputs_embeds"].shape) == (1, 6 + len("hello there"), s.hidden)
    assert tuple(kw["tts_pad_embed"].shape) == (1, 1, s.hidden)
    assert talker.generate is original  # the official method is back
    assert Sampling.from_kwargs(kw) == Sampling.greedy(processor=False)
    # the same text gives the same prompt; another text another one
    assert torch.equal(probe.prompt("hello there", "vivian", "english")["inputs_embeds"], kw["inputs_embeds"])
    assert probe.prompt("good morning", "vivian", "english")["inputs_embeds"].shape[1] == 6 + len("good morning")


def test_prompt_refuses_what_the_reference_refuses():
    tts = syn.make_hf_tts("tiny", seed=3)
    probe = Qwen3Fast(tts, graphs=False)
    gcv = tts.generate_custom_voice

    def padded(text, speaker, language, **gen):  # a batch with padding: the attention mask is not all ones
        talker = tts.model.talker
        orig = talker.generate

        def wrap(**kw):
            kw["attention_mask"] = kw["attention_mask"].clone()
            kw["attention_mask"][0, 0] = 0
            return orig(**kw)

        talker.generate = wrap
        try:
            return gcv(text, speaker, language, **gen)
        finally:
            talker.generate = orig

    tts.generate_custom_voice = padded
    with pytest.raises((ValueError, RuntimeError)):
        probe.prompt("hi", "vivian", "english")
    tts.generate_custom_voice = lambda **kw: None  # never reaches the talker
    with pytest.raises(RuntimeError):
        probe.prompt("hi", "vivian", "english")


def test_engine_cache_is_a_view_the_hf_modules_write_into():
    """The transformers cache object built over the engine's [layers, nkv, max_len, 128] tensors: a prompt run
    through Qwen3Model writes its keys and values there (bf16 cache under an fp32 model), the hidden states match
    those of the same model over a fresh DynamicCache, and seek(0) rewinds the write position."""
    from transformers import DynamicCache

    from sokutou_amd.kernels import _engine_kv_cache

    name, seed, L, max_len = "tiny", 5, 12, 40
    s = syn.workload_shape(name)
    model = syn.hf_talker_model(seed, s)
    emb = torch.from_numpy(syn.prompt_embeds(seed, s, L))
    kc = torch.zeros((s.n_layers, s.nkv, max_len, 128), dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    cache = _engine_kv_cache(model.config, max_len, kc, vc)
    ref_cache = DynamicCache()
    with torch.no_grad():
        out = model(inputs_embeds=emb, past_key_values=cache, cache_position=torch.arange(L), use_cache=True)
        ref = model(inputs_embeds=emb, past_key_values=ref_cache, cache_position=torch.arange(L), use_cache=True)
    # the static cache attends over all max_len positions (the rest masked), the dynamic one over L: the same
    # values up to summation order
    a, b = out.last_hidden_state, ref.last_hidden_state
    assert float((a - b).abs().max() / b.abs().max()) < 1e-5
    for i, layer in enumerate(ref_cache.layers):
        k, v = layer.keys[0].to(torch.bfloat16), layer.values[0].to(torch.bfloat16)
        if i == 0:  # same input rows: the same bits
            assert torch.equal(kc[i, :, :L], k) and torch.equal(vc[i, :, :L], v)
        else:  # the inputs differ by summation order: within one bf16 rounding
            assert float((kc[i, :, :L].float() - k.float()).abs().max()) <= 1e-2 * float(k.float().abs().max())
            assert float((vc[i, :, :L].float() - v.float()).abs().max()) <= 1e-2 * float(v.float().abs().max())
    assert float(kc[:, :, L:].abs().sum()) == 0
    cache.seek(0)
    kc.zero_()
    with torch.no_grad():
        model(inputs_embeds=emb, past_key_values=cache, cache_position=torch.arange(L), use_cache=True)
    assert float(kc[:, :, :L].abs().sum()) > 0 and float(kc[:, :, L:].abs().sum()) == 0


def test_eager_decode_is_the_tokenizers():
    tts = syn.make_hf_tts("tiny", seed=2)
    eng = Qwen3Fast(tts, graphs=False)
    codes = torch.randint(0, syn.workload_shape("tiny").vocab, (37, 1))
    wav, sr = eng.decode(codes)
    ref, rsr = tts.model.speech_tokenizer.decode([{"audio_codes": codes}])
    assert sr == rsr == 24000 and np.array_equal(wav, ref[0]) and wav.size == 37 * 40


# what qwen3/serve.py, bench.py, check.py and prof_frame.py read from the engine
CALLER_METHODS = ("capture", "generate_codes", "synth", "prompt", "warm_prefill", "warm_decode", "decode",
                  "teacher_logits", "weight_bytes")
CALLER_ATTRS = ("stats", "graph", "s", "talker", "tcache", "device", "sampler", "l2_keep_mb", "l2_kept_bytes",
                "cp_pair")


def test_every_caller_method_resolves_on_the_engine_class():
    from sokutou_amd.kernels import Qwen3Kernels

    for name in CALLER_METHODS:
        assert callable(getattr(Qwen3Kernels, name, None)), name
    src = inspect.getsource(Qwen3Kernels.__init__) + inspect.getsource(Qwen3Fast.__init__)
    for name in CALLER_ATTRS:
        assert re.search(rf"self\.{name}\b[^\n=]*=", src), name
    probe = Qwen3Fast(syn.make_hf_tts("tiny", seed=1), graphs=False)
    for name in ("stats", "graph", "s", "talker", "tcache", "device"):
        assert hasattr(probe, name), name
