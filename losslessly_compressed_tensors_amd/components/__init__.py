"""Training integration: autograd layers whose saved activations and weights
are held compressed, and optimizers whose momentum is (``LCT/components/``)."""
