"""``dsl_splat.runtime``: ``gradients`` of the HIP build (the launch path itself is the C ABI)."""
