// D4 kernels (added below)
