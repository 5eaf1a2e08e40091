"""CPU oracle for the int4-KV decode-attention path.

TEST INFRASTRUCTURE ONLY. Nothing in the shipped package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker or
the timed CPU baseline -- never as the thing measured or shipped.
"""
