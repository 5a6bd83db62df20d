"""Pricing-scan operators (MI355X HIP kernels behind the reference's ScanExtension interface)."""
