"""The reference's hot-path demo kernels (kernel/{matmul,conv2d,flash_attention}/*.py) as
kernel identities for the gfx950 backend: same module layout, function names, parameter
order and seeded static constants. Their bodies are DSL programs in the reference; here
``dsl_run(kernel, args, "gfx950-lowering")`` recognises them and runs the CDNA4 kernels."""
