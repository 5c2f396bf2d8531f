"""CPU oracle of the flashcodec KV-codec hot path — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker of the HIP kernels.  The flashcodec_amd package never
imports, links or calls anything here.
"""
