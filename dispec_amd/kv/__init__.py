"""Paged KV storage: host block metadata plus the HBM pool driven by HIP kernels."""
