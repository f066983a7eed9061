"""Op library with the Python signatures of the reference's engine/kernels package."""
