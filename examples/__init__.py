"""Examples built on the codec."""
