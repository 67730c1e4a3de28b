"""lmoe -- MI355X-native LatentMoE expert hot path.

Host side of the path: Python on PyTorch-ROCm calling hand-written gfx950 HIP
kernels through the C-ABI library ``liblmoe.so`` (declared in
``include/lmoe.h``).  Submodules:

  config    LatentMoEConfig / LatentMoEWeights (reference L2 types)
  _lib      ctypes binding of liblmoe.so (fails loudly when it is missing)
  ops       reference-shaped operators: ragged_dot, _router_gate,
            filter_and_pad_to_shard[_jittable], _combine_shard_contribution, ...
  forward   latent_moe_forward family
  loader    MXFP4 expert weights from safetensors checkpoints
  kernel_bench  per-kernel timing helpers
  workloads seeded synthetic inputs for the BASELINE configs
"""

from .config import (LatentMoEConfig, LatentMoEWeights, kimi_k3_config,  # noqa: F401
                     mosaic_correctness_config, single_chip_kimi_k3_config, toy_config)
