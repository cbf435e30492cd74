"""CPU oracle for M*'s ragged paged-attention path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the path
that ``mstar_amd`` implements on MI355X: page allocation and batch packing
(``mstar/engine/kv_store.py``, ``mstar/engine/cache_manager.py``), the
per-token page map and paged append (``mstar/utils/flashinfer_utils.py``), and
paged GQA attention with split-KV merging (FlashInfer semantics as M* uses
them, checked the way the reference's own tests check them:
``test/modular/test_pi05_reference_equivalence.py:158-185, 625-640``).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the CPU baseline.
The product path (``mstar_amd``) never imports it and has no CPU fallback.

Pinning (see ``tests/test_oracle_*.py``): every function here is checked
against an independent derivation — brute-force per-token simulation,
invariants, hand-computed known answers, torch's
``scaled_dot_product_attention`` and an exhaustive search over the 256 fp8
code points — not against a retyped copy of its own formula.
FlashInfer itself (``flashinfer-python>=0.6.4``, ``pyproject.toml:48``, no
exact pin) is not vendored and not installed, so its accumulation order and
split-KV schedule are not reproduced: attention parity is to a tolerance
against fp32, as the north star specifies.
"""
