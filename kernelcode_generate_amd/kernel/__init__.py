"""The hot-path demo kernels as DSL programs for the gfx950 backend, one program per
family (`matmul/tiled.py`, `conv2d/tiled.py`, `flash_attention/tiled.py`) and, in the
reference's module layout (kernel/{matmul,conv2d,flash_attention}/inputs_*.py), the demo
entry points with the reference demos' names, parameters and seeded constants, each a
call of its family's program. ``dsl_run(kernel, args, "gfx950-lowering")`` builds the IR
from the Python source, fuses a recognised nest onto a hand-written CDNA4 kernel or runs
it operation by operation."""
