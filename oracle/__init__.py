"""CPU oracle for the decode-layer hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (and, for CPU timing, in plain C under ``oracle/c``), the reference's CPU oracle for
the decode layer: the storage-format codecs and dequantizers (``monolith/formats``), the layer math of the
``monolith/nn`` torch ``forward`` oracles, and the numerics gates of ``monolith/bench.py``. Every function cites the
reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import, call or link
anything here, and only as the checker (or the timed CPU baseline). The product path
(``lithos-metal_amd/monolith_mi355``) never imports it and has no CPU fallback.

Pinning (what makes each function trustworthy, beyond being a restatement):

* ``fp``: the known answers of the reference's ``tests/contract/test_fp_codes.py`` plus brute force over every code
  (``tests/test_oracle_formats.py``).
* ``formats``: the reference's per-element NVFP4 formula test and INT4 closed form, quantize idempotence / bounded
  drift, and golden vectors written by the reference's own quantizers (``tests/golden``).
* ``nn``: golden vectors written by the reference's torch oracles (``tests/golden/make_golden.py``) for the GDN mixer,
  the attention step, the MoE route/forward, RMSNorm and the gated MLP, plus closed-form invariants (a softmax row
  sums to one, a delta-rule step on a zero state equals ``β·v·kᵀq``, RoPE preserves pair norms).
* ``kv``: the int8 KV-cache codec is defined by this build (the reference keeps a BF16 cache); it is pinned by a
  brute-force round-trip bound and exact integer identities, not by a reference vector.
"""
