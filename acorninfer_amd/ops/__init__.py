"""Drop-in operators for acorninfer/ops (HIP kernels on gfx950)."""
