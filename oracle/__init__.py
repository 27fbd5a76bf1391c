"""CPU oracle of the EstudioCanciones per-frame decode path (numpy).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package may import this module; only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the checker (or, for the CPU baseline, as the timed CPU restatement).

Every function restates the reference's algorithm with its rounding points and cites the
reference file:line it follows (paths relative to the EstudioCanciones repository):

    numerics.py  fp16 / bf16 rounding helpers
    quant.py     q8_rows                      app/convert_final.py:17-21
    rope.py      rope_cache, apply_rope       app/engine.py:28-53
    kernels.py   _gemv8/int8_mm, _rms, _rope_cache, _attn, _attn_combine, _silu_mul,
                 Emb                          app/kernels.py:11-180, app/engine.py:89-104
    model.py     Stack.decode, _sample, _guided, _frame_fast, _step
                                              app/engine.py:156-211, :291-349

How each function is pinned (the reference ships no tests or golden vectors) is recorded
in the tests under tests/test_oracle_*.py: closed forms, invariants, brute force on tiny
inputs and special cases chosen so that a plausible slip (dropped term, wrong sign or
index, transposed operand, wrong rounding mode) fails at least one of them.
"""
