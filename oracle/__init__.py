"""CPU restatement of the reference Depthformer decode path -- test infrastructure only.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, as the checker and the timed CPU baseline; the product
(``magenta-realtime-mlx-cpp_amd/``) never imports it.
"""
