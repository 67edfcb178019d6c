"""CPU restatement of the reference's routed-expert MoE arithmetic.

TEST INFRASTRUCTURE ONLY.  Nothing under ``cachalot_amd/`` imports this
package.  It is imported by ``tests/`` (as the parity checker),
``__graft_entry__.smoke()`` (to check one small GPU invocation) and
``bench.py``'s ``cpu_baseline`` leg (timed as the reference's CPU path, a
NumPy "port").  It is never the thing measured on the GPU and never a
fallback for the HIP library.

Modules and the reference behaviour each restates (paths relative to the
reference checkout):

* ``bf16``     bf16 round-to-nearest-even, the cast MLX's ``astype(bfloat16)`` does.
* ``synth``    the seeded synthetic bank generator (twin of the GPU fill kernel).
* ``fp4``      ``src/cachalot/model/fp4.py:5-109`` (E2M1 table, E8M0, nibble order).
* ``affine2``  MLX affine 2-bit layout (``benchmarks/quant_affine.py:60-66``) and the
               qmv group formula (``src/cachalot/minimax/codes_qmv.py:86-100``).
* ``router``   ``src/cachalot/model/router_mlx.py:16-118``,
               ``router_fused_metal.py:61-108`` (tie rule / order),
               ``minimax/language.py:280-292`` (sigmoid, rank order).
* ``experts``  ``moe_fused_metal.py:189-233`` (FP4 decode), ``expert_affine.py:65-152``
               (2-bit decode), ``fp4_sgmm_metal.py:203-333`` (FP4 prefill).
* ``dispatch`` ``moe_prefill_grouped.py:199-245,464-467,526-545`` (permute / combine).
"""
