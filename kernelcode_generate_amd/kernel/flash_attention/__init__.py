"""Demo kernels of this family (see the package docstring)."""
