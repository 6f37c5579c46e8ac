"""``dsl_splat.primitives``: ``tiling`` and ``spherical_harmonics`` of the HIP build."""
