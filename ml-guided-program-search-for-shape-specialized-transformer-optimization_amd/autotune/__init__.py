"""Launch-parameter search for the gfx950 HIP programs."""
