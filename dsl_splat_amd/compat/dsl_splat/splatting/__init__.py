"""``dsl_splat.splatting``: ``binning``, ``cameras`` and ``geometry`` of the HIP build."""
