"""sokutou_amd: MI355X (gfx950) Qwen3-TTS talker decode step behind the reference's Qwen3Kernels surface.

Modules: ``kernels`` (Qwen3Kernels, _Lin, _Stack), ``fast`` (Sampling, _sample, Qwen3Fast), ``sampler``
(FusedSampler), ``synthetic`` (seeded random-init talker), ``build`` (hipcc build of libsokutou_amd.so) and
``_lib`` (ctypes binding of the C-ABI in include/sokutou_amd.h).
"""

__version__ = "0.1.0"
