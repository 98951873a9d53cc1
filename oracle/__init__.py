"""CPU oracle for the Voyager quantization hot path.

TEST INFRASTRUCTURE ONLY: a restatement of the reference's CPU algorithm used
as the parity checker and as the timed CPU baseline.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it; the product package never does.
"""
