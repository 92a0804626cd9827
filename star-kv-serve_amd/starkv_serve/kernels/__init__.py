"""Decode and cache-write kernels (HIP, gfx950) behind the reference's kernel API."""
