"""Active-support cost evaluation (SDDMM) on MI355X."""
