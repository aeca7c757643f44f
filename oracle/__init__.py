"""CPU oracle of voxwerk's token sampler — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import this
package, and only as the checker or the timed CPU baseline; the product path never does.

- ``oracle.ref``: ctypes wrapper of ``libvxs_oracle.so`` (C restatement, ``vxs_oracle.c``).
- ``oracle.sampler_np``: an independent numpy/Python restatement used to cross-check the C one.
- ``oracle.embedding_np``: the embedding lookups of sampled ids (bf16 widening, frame sums).
- ``oracle.head_np``: the logit heads (exact dot products and the fp32 error bound).
"""
