"""The real-model path on the GPU with an HF-shaped stand-in for qwen-tts (``synthetic.make_hf_tts``): synth()
end to end (prompt interception, the prefill through the talker's Hugging Face modules into the shared cache, the
frames, the speech-tokenizer decode), prefill graphs against the eager prefill, decode graphs against the
tokenizer's own decode, and no recording during synth after warm_prefill / warm_decode (qwen3/serve.py:99-107)."""

import numpy as np
import pytest
import torch

from sokutou_amd import synthetic as syn
from sokutou_amd.fast import Sampling

pytestmark = pytest.mark.gpu
TEXT, SPEAKER, LANG = "the quick brown fox", "vivian", "english"


def _engine(gpu, graphs=True, frame_kernel=True, max_cache=96):
    from sokutou_amd.kernels import Qwen3Kernels

    tts = syn.make_hf_tts("small06b", seed=6, device=gpu)
    eng = Qwen3Kernels(tts, Sampling.greedy(processor=False), max_cache=max_cache, wd="i8row", graphs=graphs,
                       sampler="fused", suppress_tail=0, frame_kernel=frame_kernel)
    return eng, tts


@pytest.mark.parametrize("frame_kernel", [True, False])
def test_synth_end_to_end_with_warm_graphs(gpu, frame_kernel):
    """capture, warm_prefill, warm_decode, then synth: codes equal those of an engine without graphs (eager prefill
    and frames), the waveform equals the tokenizer's own decode of those codes, and synth records no graph."""
    print(f"small06b stand-in: synth with warm graphs ({'frame kernel' if frame_kernel else 'per-op kernels'})",
          flush=True)
    eng, tts = _engine(gpu, graphs=True, frame_kernel=frame_kernel)
    L = int(eng.prompt(TEXT, SPEAKER, LANG)["inputs_embeds"].shape[1])
    assert eng.capture() > 0
    assert eng.warm_prefill([L]) > 0 and eng.warm_decode() > 0
    wav, sr, codes = eng.synth(TEXT, SPEAKER, LANG, max_frames=24)
    torch.cuda.synchronize()
    assert not any(k in eng.stats for k in ("prefill_capture_sec", "decode_capture_sec")), eng.stats
    assert set(("prompt", "generate", "decode")) <= set(eng.stats)
    assert codes.shape == (24, 1) and eng.stats["prompt_tokens"] == L
    ref_eng, _ = _engine(gpu, graphs=False, frame_kernel=frame_kernel)
    ref_codes = ref_eng.generate_codes(ref_eng.prompt(TEXT, SPEAKER, LANG), max_frames=24)
    assert torch.equal(codes, ref_codes)
    ref_wav, ref_sr = tts.model.speech_tokenizer.decode([{"audio_codes": codes}])
    assert sr == ref_sr and wav.shape == ref_wav[0].shape
    np.testing.assert_allclose(wav, ref_wav[0], rtol=0, atol=1e-6)


def test_prefill_graph_equals_eager_prefill(gpu):
    """The recorded prefill of one prompt length, replayed: the cache rows [0, L) and the last hidden state match
    the eager prefill's (within one bf16 rounding of the stored keys and values: the attention kernel recorded in a
    graph may sum in another order), and the first code and the frame state are the same; twice in a row."""
    print("small06b stand-in: prefill graph replay against the eager prefill", flush=True)
    a, _ = _engine(gpu, graphs=True)
    b, _ = _engine(gpu, graphs=False)
    kw = a.prompt(TEXT, SPEAKER, LANG)
    L = int(kw["inputs_embeds"].shape[1])
    for _ in range(2):
        a._start(kw)
        b._start(kw)
        torch.cuda.synchronize()
        assert L in a._pf and not b._pf
        for x, y in ((a.kc, b.kc), (a.vc, b.vc)):
            d = float((x[:, :, :L].float() - y[:, :, :L].float()).abs().max())
            print(f"  cache max abs diff {d:.3e}", flush=True)
            assert d <= 1e-2 * float(y[:, :, :L].float().abs().max())
        d = float((a.ph32 - b.ph32).abs().max() / b.ph32.abs().max())
        print(f"  last hidden max rel diff {d:.3e}", flush=True)
        assert d < 1e-4
        for x, y in ((a.id0, b.id0), (a.next_id0, b.next_id0), (a.seen, b.seen), (a.ngen, b.ngen), (a.pos, b.pos)):
            assert torch.equal(x, y)
        assert int(a.pos.item()) == L and int(a.ngen.item()) == 1


def test_decode_graphs_match_the_tokenizer(gpu):
    """Bucketed decode graphs (segments zero-padded to a bucket) against the tokenizer's decode of the whole code
    sequence, for lengths inside one bucket, on a bucket edge and across the 300-frame chunking."""
    print("small06b stand-in: decode graphs against the tokenizer", flush=True)
    eng, tts = _engine(gpu, graphs=True)
    g = torch.Generator().manual_seed(1)
    for F in (5, 16, 37, 300, 341):
        codes = torch.randint(0, eng.V, (F, 1), generator=g).to(gpu)
        wav, sr = eng.decode(codes)
        ref, _ = tts.model.speech_tokenizer.decode([{"audio_codes": codes}])
        assert wav.shape == ref[0].shape == (F * 40,)
        np.testing.assert_allclose(wav, ref[0], rtol=0, atol=1e-6)


def test_engine_has_every_attribute_the_callers_use(gpu):
    eng, _ = _engine(gpu)
    for name in ("capture", "generate_codes", "synth", "prompt", "warm_prefill", "warm_decode", "decode",
                 "teacher_logits", "weight_bytes", "stats", "graph", "s", "talker", "tcache", "device", "sampler",
                 "l2_keep_mb", "l2_kept_bytes", "cp_pair"):
        assert hasattr(eng, name), name
    assert eng.tcache is not None and eng.tcache.layers[0].keys.data_ptr() == eng.kc.data_ptr()
