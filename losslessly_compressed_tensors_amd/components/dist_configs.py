"""Default codebooks of the training integration (``LCT/components/dist_configs.py:4-35``).

Weights and activations use the Laplace family; momentum the empirical family
with a small zero mass, and a half-zero mass on Muon's first step, when the
momentum is mostly exact zeros.  Post-ReLU activations put half their mass on
zero.
"""
from ..comp_format import DistType, Distribution, NoiseLevel

weight_dist = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN)
momentum_dist = Distribution(DistType.EMPIRICAL, noise_level=NoiseLevel.CLEAN, zero_prob=0.02)
momentum_first_dist = Distribution(DistType.EMPIRICAL, noise_level=NoiseLevel.CLEAN,
                                   zero_prob=0.5)
act_dist = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN)
act_relu_dist = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN, zero_prob=0.5)
