"""Dequantization, fused GEMV and row-window streaming on the HIP library."""
