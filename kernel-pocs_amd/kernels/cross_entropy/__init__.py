"""Cross-entropy on MI355X (drop-in for kernels/cross_entropy)."""
