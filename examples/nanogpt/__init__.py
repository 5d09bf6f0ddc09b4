"""GPT-2-small training with compressed weights, activations and momentum."""
