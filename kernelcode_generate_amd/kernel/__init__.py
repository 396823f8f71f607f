"""The reference's hot-path demo kernels (kernel/{matmul,conv2d,flash_attention}/*.py) as
DSL programs for the gfx950 backend: same module layout, function names, parameter order,
seeded static constants and loop nests. ``dsl_run(kernel, args, "gfx950-lowering")``
builds their IR from the Python source, fuses a recognised nest onto a hand-written CDNA4
kernel or runs it operation by operation."""
