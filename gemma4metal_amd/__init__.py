"""MI355X-native (gfx950) int4-KV decode attention: the ``turboquant`` hot path
of svv232/gemma4metal rebuilt as hand-written HIP behind a C ABI.

    from gemma4metal_amd import turboquant as tq
    out = tq.sdpa_int4(q, kq, ks, kb, vq, vs, vb, gqa_factor=2)
"""
from . import turboquant  # noqa: F401

__all__ = ["turboquant"]
