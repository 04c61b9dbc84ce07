"""Hand-written gfx950 kernels behind the plan API (loaded lazily)."""
