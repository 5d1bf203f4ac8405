"""kadconv: KAD-Conv with gfx950 HIP kernels behind the reference's API."""
