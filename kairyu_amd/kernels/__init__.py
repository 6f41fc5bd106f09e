"""Host wrappers of the HIP kernels (mirror of ``kairyu.kernels``)."""
