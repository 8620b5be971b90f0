"""The C-ABI library loads on a machine without a GPU, exports every function declared in
include/sokutou_amd.h, and rejects bad shapes before launching anything. No kernel is launched here."""

import ctypes
import re

import pytest

from sokutou_amd import _lib


def _declared():
    text = _lib.HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    names = _declared()
    assert "sk_attn" in names and "sk_rms_gemv" in names
    for n in names:
        assert hasattr(L, n), n
    assert set(names) <= set(_lib._SIGS), "every declared entry point has a ctypes signature"


def test_version_string():
    assert b"gfx950" in _lib.load().sk_version()


def test_workspace_size():
    L = _lib.load()
    # the error word, a counter per kv head and the partials (m, l, o[128]) of both q heads of every split: 8 splits
    # at 1024 positions (one per 128, at least 8), 16 at 4096 (at most 16), one below 129
    assert L.sk_attn_workspace_size(16, 8, 1024) >= 8 * 2 * 8 * 130 * 4 + 8 * 4 + 4
    assert L.sk_attn_workspace_size(16, 8, 4096) >= 8 * 2 * 16 * 130 * 4 + 8 * 4 + 4
    assert L.sk_attn_workspace_size(16, 8, 16) >= 8 * 2 * 130 * 4 + 8 * 4 + 4
    assert L.sk_attn_workspace_size(16, 0, 16) == 0


@pytest.mark.parametrize("N,K", [(64, 1000), (0, 1024), (64, 16384)])
def test_gemv_rejects_bad_shapes_without_launching(N, K):
    L = _lib.load()
    dummy = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = L.sk_gemv(dummy, dummy, dummy, None, dummy, N, K, 0, 0, 1, None)
    assert rc == _lib.SK_EINVAL
    assert b"sk_gemv" in L.sk_last_error()
    with pytest.raises(ValueError):
        _lib.check(rc, "sk_gemv")


def test_attn_rejects_bad_head_ratio():
    L = _lib.load()
    d = ctypes.c_void_p(256)
    rc = L.sk_attn(d, d, d, 1e-6, d, d, d, None, 0, 64, 12, 8, d, d, 1 << 20, 0, None)
    assert rc == _lib.SK_EINVAL


def test_sample_rejects_bad_arguments_without_launching():
    L = _lib.load()
    d = ctypes.c_void_p(256)
    assert L.sk_sample(d, 5000, 1.0, 0, 0, None, 1.0, None, None, 0, -1, None, None, d, 0, None, None, None) == _lib.SK_EINVAL
    # sampling needs the device seed and counter, and a positive temperature
    assert L.sk_sample(d, 100, 1.0, 50, 1, None, 1.0, None, None, 0, -1, None, d, d, 0, None, None, None) == _lib.SK_EINVAL
    assert L.sk_sample(d, 100, 0.0, 50, 1, None, 1.0, None, None, 0, -1, d, d, d, 0, None, None, None) == _lib.SK_EINVAL
    rc = L.sk_sample(d, 100, -2.0, 50, 1, None, 1.0, None, None, 0, -1, d, d, d, 0, None, None, None)
    assert rc == _lib.SK_EINVAL
    with pytest.raises(ValueError):
        _lib.check(rc, "sk_sample")


def test_cp_frame_rejects_bad_shapes_without_launching():
    import ctypes

    from sokutou_amd import _lib

    L = _lib.load()
    d = _lib.SkCpDesc(n_layers=5, hidden=1024, inter=3072, nq=16, nkv=8, vocab=3000, n_positions=16)
    assert L.sk_cp_frame(ctypes.byref(d), None) == _lib.SK_EUNSUPPORTED
    d.vocab = 2048
    assert L.sk_cp_frame(ctypes.byref(d), None) == _lib.SK_EINVAL  # null pointers
    d.n_positions = 1
    assert L.sk_cp_frame(ctypes.byref(d), None) == _lib.SK_EUNSUPPORTED


def test_cp_frame_checks_the_projection_without_launching():
    """A projected code predictor: 2048-wide inputs only, its weights (and scales, for int8) present, unpaired."""
    L = _lib.load()
    dv = ctypes.c_void_p(256)
    c = _lib.SkCpDesc(n_layers=5, hidden=1024, inter=3072, nq=16, nkv=8, vocab=2048, n_positions=16,
                      wd=_lib.WD["i8row"], ct=_lib.CT["bf16"], eps=1e-6, layers=dv, norm=dv, rope=dv, x0=dv, id0=dv,
                      emb0_rows=3072, emb=dv, head_w=dv, head_s=dv, codes=dv, workspace=dv,
                      workspace_bytes=int(L.sk_cp_workspace_size(1024, 3072, 0)), proj_in=1536, proj_w=dv, proj_s=dv)
    assert L.sk_cp_frame(ctypes.byref(c), None) == _lib.SK_EUNSUPPORTED
    c.proj_in, c.proj_s = 2048, None
    assert L.sk_cp_frame(ctypes.byref(c), None) == _lib.SK_EINVAL  # int8 projection without its scales
    c.proj_s, c.pair = dv, 1
    assert L.sk_cp_frame(ctypes.byref(c), None) == _lib.SK_EUNSUPPORTED
    assert b"unpaired" in L.sk_last_error()


def test_frame_workspace_holds_trace_and_placed_cell_region():
    """Control words (256 bytes), the trace stamps (256 workgroups x 2 roles x 32 layers x 16 events x 8 bytes),
    then a 2 MB cell region at the first 2 MB boundary after them (2 MB of slack): one size for the talker at both
    shapes and every code predictor (paired or projected), whose cells all fit the region's 64 x 512 cells; a shape
    whose cells would not fit gets 0."""
    L = _lib.load()
    want = 256 + 256 * 2 * 32 * 16 * 8 + 2 * (2 << 20)
    assert L.sk_talker_workspace_size(1024, 3072) == want
    assert L.sk_talker_workspace_size(2048, 6144) == want
    assert L.sk_cp_workspace_size(1024, 3072, 0) == want
    assert L.sk_cp_workspace_size(1024, 3072, 1) == want
    assert L.sk_cp_workspace_size(0, 3072, 1) == 0
    assert L.sk_talker_workspace_size(4096, 12288) == 0  # 35840 cells > 32768


def test_frames_place_checks_arguments_before_the_device():
    """sk_frames_place refuses a null or short workspace before it queries the device."""
    L = _lib.load()
    assert L.sk_frames_place(None, 1 << 30, None) == _lib.SK_EINVAL
    assert L.sk_frames_place(ctypes.c_void_p(256), int(L.sk_talker_workspace_size(1024, 3072)) - 1,
                             None) == _lib.SK_EWORKSPACE
    assert b"too small" in L.sk_last_error()


def test_batched_entry_points_reject_bad_shapes_without_launching():
    import ctypes

    L = _lib.load()
    d = ctypes.c_void_p(256)
    assert L.sk_batch_terms() in (1, 2, 3)
    # K not a supported length, N not a multiple of 16, SwiGLU with N % 32 != 0, accumulate without its outputs
    W = (d, 1 << 20, None)  # workspace, its size, stream
    assert L.sk_bgemm(d, None, 0, 1e-6, d, d, 64, 1000, 0, d, None, None, None, None, *W) == _lib.SK_EINVAL
    assert L.sk_bgemm(d, None, 0, 1e-6, d, d, 40, 1024, 0, d, None, None, None, None, *W) == _lib.SK_EINVAL
    assert L.sk_bgemm(d, None, 0, 1e-6, d, d, 48, 1024, 1, None, d, None, None, None, *W) == _lib.SK_EINVAL
    assert L.sk_bgemm(d, None, 0, 1e-6, d, d, 64, 1024, 2, d, None, None, None, None, *W) == _lib.SK_EINVAL
    assert L.sk_bgemm(d, d, 0, 1e-6, d, d, 64, 1024, 0, d, None, None, None, None, *W) == _lib.SK_EINVAL
    assert L.sk_tile_weights(d, d, 40, 128, None) == _lib.SK_EINVAL
    # a workspace smaller than the split-K partials of the 1.7B down projection
    need = L.sk_bgemm_workspace_size(2048, 6144)
    assert need > 0 and L.sk_bgemm_workspace_size(40, 1024) == 0
    assert L.sk_bgemm(d, None, 0, 1e-6, d, d, 2048, 6144, 0, d, None, None, None, None, d, need - 256, None) == \
        _lib.SK_EWORKSPACE
    ws = L.sk_batch_workspace_size(2048, 6144, 16, 8, 3072)
    assert ws > 16 * 8 * 2 * 32 * 130 * 4  # attention partials of 16 streams x 8 kv heads x 32 splits
    desc = _lib.SkBatchDesc(n_layers=28, hidden=2048, inter=6144, nq=16, nkv=8, vocab=3072, batch=17, max_len=2100)
    assert L.sk_batch_frame(ctypes.byref(desc), None) == _lib.SK_EINVAL  # batch > 16
    desc.batch = 16
    assert L.sk_batch_frame(ctypes.byref(desc), None) == _lib.SK_EINVAL  # null pointers
    desc.max_len = 5000
    assert L.sk_batch_embed(ctypes.byref(desc), None) == _lib.SK_EINVAL  # cache longer than the attention supports


def test_frame_kernels_reject_sampling_without_seed_or_temperature():
    """Sampled picks inside the persistent kernels need the device seed and counter and inv_temp > 0; the
    checks run before the kernel is launched (and before the device is queried)."""
    L = _lib.load()
    d = ctypes.c_void_p(256)
    ws = int(L.sk_talker_workspace_size(1024, 3072))
    t = _lib.SkTalkerDesc(n_layers=2, hidden=1024, inter=3072, nq=16, nkv=8, vocab=3072, max_len=64,
                          wd=_lib.WD["i8row"], ct=_lib.CT["bf16"], eps=1e-6, layers=d, norm=d, head_w=d, head_s=d,
                          emb=d, rope=d, id0=d, pos=d, workspace=d, workspace_bytes=ws, do_sample=1, inv_temp=1.0,
                          top_k=50, seed=None, counter=d)
    assert L.sk_talker_frames(ctypes.byref(t), 1, None) == _lib.SK_EINVAL
    assert b"sampling" in L.sk_last_error()
    t.seed, t.inv_temp = d, 0.0
    assert L.sk_talker_frames(ctypes.byref(t), 1, None) == _lib.SK_EINVAL
    c = _lib.SkCpDesc(n_layers=5, hidden=1024, inter=3072, nq=16, nkv=8, vocab=2048, n_positions=16,
                      wd=_lib.WD["i8row"], ct=_lib.CT["bf16"], eps=1e-6, layers=d, norm=d, rope=d, x0=d, id0=d,
                      emb0_rows=3072, emb=d, head_w=d, head_s=d, codes=d, workspace=d,
                      workspace_bytes=int(L.sk_cp_workspace_size(1024, 3072, 0)), do_sample=1, inv_temp=1.25,
                      top_k=40, seed=d, counter=None)
    assert L.sk_cp_frame(ctypes.byref(c), None) == _lib.SK_EINVAL
    assert b"sampling" in L.sk_last_error()


def test_code_predictor_keep_policies_follow_the_reference_budget():
    """l2_keep_mb walks the code predictor's matrices in layer order (qwen3/kernels.py:525-542): a matrix that fits
    what is left of the budget stays cacheable and uses it up, one that does not is streamed (a later, smaller one
    may still fit); no budget keeps everything."""
    from sokutou_amd.kernels import _keep_policies

    class M:
        def __init__(self, n):
            self.n, self.pol = n, None

        def bytes(self):
            return self.n

    MiB = 2**20
    layers = [{"qkv": M(4 * MiB), "o": M(2 * MiB), "gu": M(6 * MiB), "down": M(3 * MiB)} for _ in range(2)]
    assert _keep_policies(layers, None) == 30 * MiB
    assert all(Ly[m].pol == 0 for Ly in layers for m in Ly)
    assert _keep_policies(layers, 10) == 9 * MiB  # qkv 4 + o 2 kept, gu 6 > 4 left streamed, down 3 kept
    assert [layers[0][m].pol for m in ("qkv", "o", "gu", "down")] == [0, 0, 1, 0]
    assert [layers[1][m].pol for m in ("qkv", "o", "gu", "down")] == [1, 1, 1, 1]
    assert _keep_policies(layers, 0) == 0 and all(Ly[m].pol == 1 for Ly in layers for m in Ly)
