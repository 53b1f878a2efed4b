"""CPU oracle and CPU baseline of the PESQ pipeline.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, never by the shipped package.
"""
