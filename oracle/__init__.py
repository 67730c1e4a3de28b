"""CPU oracle for the LatentMoE expert hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package may import, call or
link anything under ``oracle/``.  The only permitted users are ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, and
only as the checker / the timed CPU restatement, never as the thing that is
shipped or measured on the GPU.

``lmoe_oracle`` restates, in numpy, the algorithms of the reference
(``05_ragged_dot_on_tpu/kimi_k3_latent_moe_reference.py`` and friends); each
function cites the reference ``file:line`` it follows.
"""
