"""Drop-in replacements for the reference's ``ops/triton/*`` entry points (HIP kernels)."""
