"""ctypes binding of ``libsokutou_amd.so`` (the C-ABI declared in ``include/sokutou_amd.h``).

torch is imported before the library is opened: torch bundles its own HIP runtime with the same soname
(``libamdhip64.so.7``), so the dynamic loader resolves the library against that one runtime and the stream
handles torch hands out (``torch.cuda.current_stream().cuda_stream``) are valid inside the library.
There is no fallback: if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must be loaded first, see above)

LIB_PATH = Path(__file__).resolve().parent / "libsokutou_amd.so"
HEADER = Path(__file__).resolve().parent.parent / "include" / "sokutou_amd.h"

SK_OK, SK_EINVAL, SK_ELAUNCH, SK_EUNSUPPORTED, SK_EWORKSPACE, SK_EDEVICE = 0, -1, -2, -3, -4, -5
WD = {"i8row": 0, "i8g32": 1, "bf16": 2, "f32": 3}
CT = {"bf16": 0, "f32": 1}

_P = c_void_p
_SIGS = {
    "sk_version": (ctypes.c_char_p, []),
    "sk_last_error": (ctypes.c_char_p, []),
    "sk_device_check": (c_int, []),
    "sk_rms_gemv": (c_int, [_P, _P, c_float, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P]),
    "sk_gemv": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P]),
    "sk_rmsnorm": (c_int, [_P, _P, c_float, _P, c_int, _P]),
    "sk_embed": (c_int, [_P, _P, _P, c_int, c_int, _P]),
    "sk_talker_in": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _P]),
    "sk_attn_workspace_size": (c_int64, [c_int, c_int, c_int]),
    "sk_attn": (c_int, [_P, _P, _P, c_float, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P, _P, c_int64, c_int, _P]),
    "sk_attn_noalloc": (c_int, [_P, _P, _P, c_float, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P, _P, c_int, _P]),
    "sk_sample": (c_int, [_P, c_int, c_float, c_int, c_int, _P, c_float, _P, _P, c_int, c_int, _P, _P, _P, c_int, _P,
                          _P, _P]),
}



class SkLayerDesc(ctypes.Structure):
    """Mirror of ``sk_layer_desc`` (include/sokutou_amd.h)."""
    _fields_ = [(n, c_void_p) for n in ("qkv_w", "qkv_s", "o_w", "o_s", "gu_w", "gu_s", "down_w", "down_s", "in_norm",
                                        "post_norm", "qn", "kn", "kc", "vc")]


class SkTalkerDesc(ctypes.Structure):
    """Mirror of ``sk_talker_desc`` (include/sokutou_amd.h)."""
    _fields_ = [("n_layers", c_int), ("hidden", c_int), ("inter", c_int), ("nq", c_int), ("nkv", c_int),
                ("vocab", c_int), ("max_len", c_int), ("wd", c_int), ("ct", c_int), ("eps", c_float),
                ("layers", c_void_p), ("norm", c_void_p), ("head_w", c_void_p), ("head_s", c_void_p), ("emb", c_void_p),
                ("rope", c_void_p), ("id0", c_void_p), ("pos", c_void_p), ("next_id0", c_void_p), ("out", c_void_p),
                ("seen", c_void_p), ("ngen", c_void_p), ("suppress", c_void_p), ("rep_pen", c_float),
                ("min_new", c_int), ("eos", c_int), ("talker_processor", c_int), ("logits", c_void_p),
                ("layer_out", c_void_p), ("workspace", c_void_p), ("workspace_bytes", c_int64),
                ("in_tabs", c_void_p), ("in_codes", c_void_p), ("in_pad", c_void_p), ("in_groups", c_int),
                ("in_rows", c_int), ("final_out", c_void_p), ("do_sample", c_int), ("inv_temp", c_float),
                ("top_k", c_int), ("seed", c_void_p), ("counter", c_void_p)]


class SkCpDesc(ctypes.Structure):
    """Mirror of ``sk_cp_desc`` (include/sokutou_amd.h)."""
    _fields_ = [("n_layers", c_int), ("hidden", c_int), ("inter", c_int), ("nq", c_int), ("nkv", c_int),
                ("vocab", c_int), ("n_positions", c_int), ("wd", c_int), ("ct", c_int), ("eps", c_float),
                ("layers", c_void_p), ("norm", c_void_p), ("rope", c_void_p), ("x0", c_void_p), ("id0", c_void_p),
                ("emb0_rows", c_int), ("emb", c_void_p), ("head_w", c_void_p), ("head_s", c_void_p),
                ("codes", c_void_p), ("logits", c_void_p), ("layer_out", c_void_p), ("workspace", c_void_p),
                ("workspace_bytes", c_int64), ("do_sample", c_int), ("inv_temp", c_float), ("top_k", c_int),
                ("seed", c_void_p), ("counter", c_void_p), ("keep_layers", c_int), ("pair", c_int),
                ("proj_in", c_int), ("proj_w", c_void_p), ("proj_s", c_void_p), ("proj_b", c_void_p)]


class SkBatchDesc(ctypes.Structure):
    """Mirror of ``sk_batch_desc`` (include/sokutou_amd.h)."""
    _fields_ = [("n_layers", c_int), ("hidden", c_int), ("inter", c_int), ("nq", c_int), ("nkv", c_int),
                ("vocab", c_int), ("batch", c_int), ("max_len", c_int), ("eps", c_float), ("layers", c_void_p),
                ("norm", c_void_p), ("head_w", c_void_p), ("head_s", c_void_p), ("emb", c_void_p), ("rope", c_void_p),
                ("ids", c_void_p), ("pos", c_void_p), ("codes", c_void_p), ("nstep", c_void_p),
                ("max_frames", c_int), ("logits", c_void_p), ("layer_out", c_void_p), ("workspace", c_void_p),
                ("workspace_bytes", c_int64)]


_SIGS["sk_batch_terms"] = (c_int, [])
_SIGS["sk_tile_weights"] = (c_int, [_P, _P, c_int, c_int, _P])
_SIGS["sk_bgemm"] = (c_int, [_P, _P, c_int, c_float, _P, _P, c_int, c_int, c_int, _P, _P, _P, _P, _P, _P, c_int64, _P])
_SIGS["sk_bgemm_workspace_size"] = (c_int64, [c_int, c_int])
_SIGS["sk_batch_workspace_size"] = (c_int64, [c_int, c_int, c_int, c_int, c_int])
_SIGS["sk_batch_attn_workspace_size"] = (c_int64, [c_int])
_SIGS["sk_batch_attn"] = (c_int, [_P, _P, _P, c_float, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P, _P, c_int64, _P])
_SIGS["sk_batch_embed"] = (c_int, [ctypes.POINTER(SkBatchDesc), _P])
_SIGS["sk_batch_frame"] = (c_int, [ctypes.POINTER(SkBatchDesc), _P])
_SIGS["sk_talker_workspace_size"] = (c_int64, [c_int, c_int])
_SIGS["sk_talker_frames"] = (c_int, [ctypes.POINTER(SkTalkerDesc), c_int, _P])
_SIGS["sk_cp_frame"] = (c_int, [ctypes.POINTER(SkCpDesc), _P])
_SIGS["sk_cp_workspace_size"] = (c_int64, [c_int, c_int, c_int])
_SIGS["sk_frames_place"] = (c_int, [_P, c_int64, _P])

_lib = None


def load() -> ctypes.CDLL:
    """Opens the library once and declares every signature."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m sokutou_amd.build` (hipcc, gfx950)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int, name: str) -> None:
    """Raises the Python error matching an SK_* status (ValueError where the reference asserts)."""
    if rc == SK_OK:
        return
    msg = f"{name}: {load().sk_last_error().decode(errors='replace')}"
    if rc in (SK_EINVAL, SK_EWORKSPACE):
        raise ValueError(msg)
    if rc == SK_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def ptr(t) -> int | None:
    """Device address of a tensor (None for None); tensors must be contiguous, as in the reference's _ptr
    (qwen3/kernels.py:418-422)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)
