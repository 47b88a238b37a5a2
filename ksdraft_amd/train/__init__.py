"""Training-side helpers the INT8 kernels call (reference ksdraft/train)."""
