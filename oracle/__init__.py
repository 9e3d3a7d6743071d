"""CPU fp32 oracle for the CosyVoice3 Token2Wav DiT estimator path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this package: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the reference they compare against (or as the timed CPU baseline),
never as the thing measured or shipped.

``dit_oracle`` restates the reference's fp32 torch DiT (padded SDPA with
boolean masks) and its packed CFG Euler solver; ``frontend_oracle`` restates the
Flow front-end that produces the DiT inputs (token embedding, PreLookaheadLayer,
speaker projection, prompt condition).
"""
