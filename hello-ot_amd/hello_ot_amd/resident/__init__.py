"""GPU-resident HELLO driver over the MI355X hot-path kernels (hierarchy, active support, refinement loop)."""
