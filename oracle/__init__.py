"""CPU oracle for the sqrt(N) sparse-attention hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import anything from this package,
and only as the checker (or the timed CPU baseline), never as the thing that
is measured or shipped.  The product package (``cron_root_attention``) never
imports it: on a GPU it runs the HIP library or raises.

Contents: ``cra_oracle`` (fp64 restatement of the reference's forward and
relay selection, autograd backward, index-set brute force and the pair-count
work model) and ``cpu_port`` (the chunked CPU path used as the timed baseline).
"""
