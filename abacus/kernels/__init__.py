"""abacus.kernels: the cross-entropy switch of the reference (see abacus_amd.train)."""
