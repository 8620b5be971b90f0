"""CPU oracle for the Qwen3-TTS talker decode step.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or as the timed CPU baseline). The
product path (``sokutou_amd``) never imports it and has no CPU fallback.
"""
