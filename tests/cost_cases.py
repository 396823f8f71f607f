"""Run each cost-model case once on the GPU and print the modelled costs, so a hardware
counter run can be laid beside the model:

    rocprofv3 --pmc SQ_INSTS_MFMA -d <dir> -- python3 -m tests.cost_cases

Every case makes one library MFMA kernel dispatch, in the order printed, followed (for the
conv cases whose grid is small enough to split K) by a split-K reduction kernel that issues
no MFMA; inputs are generated on the host and copied, and the only other
dispatches are the HIP runtime's own copy kernels (named __amd_rocclr_*) that some
host-to-device copies use, so leaving out those and the *_splitk_reduce_kernel dispatches,
library dispatch i of the counter run is case i. Cases cover every kernel choice the model distinguishes: the
pipelined MFMA GEMM with 256- and 128-row tiles and with ragged edges, the fp32 MFMA GEMM
aligned and ragged, the fp32 split-K GEMM, the SIMT GEMM, the MFMA conv with four and with two live waves and a
ragged last row block, the implicit-GEMM conv (16-bit and fp32) and its row-piece form
(16-bit 8- and 4-pixel pieces, 3x3 and 1x1, stride 1 and 2; fp32), and the 16-bit and fp32 MFMA attention kernels for D=128 and D=64,
causal and not, with ragged query and key tails.
"""

from __future__ import annotations

import argparse
import json
import sys

from kernelcode_generate_amd import native

# (name, family, dtype, shapes, scalars): shapes are (out, in0, in1[, in2]) in the slot
# order of the family's entry; bias is always absent. No matmul case takes the split-K path;
# the two implicit-GEMM conv cases and three of the row-piece ones do (their reduce dispatch
# issues no MFMA).
CASES = (
    ("gemm_bf16_4096", "matmul", "bfloat16", ((4096, 4096), (4096, 4096), (4096, 4096)), ()),
    ("gemm_bf16_c2s_8192x1024x4096", "matmul", "bfloat16", ((8192, 1024), (8192, 4096), (4096, 1024)), ()),
    ("gemm_f16_512x768x256", "matmul", "float16", ((512, 768), (512, 256), (256, 768)), ()),
    ("gemm_bf16_ragged_1000x1000x488", "matmul", "bfloat16", ((1000, 1000), (1000, 488), (488, 1000)), ()),
    ("gemm_f32_256", "matmul", "float32", ((256, 256), (256, 256), (256, 256)), ()),
    ("gemm_f32_splitk_512x512x4096", "matmul", "float32", ((512, 512), (512, 4096), (4096, 512)), ()),
    ("gemm_f32_simt_250x250x250", "matmul", "float32", ((250, 250), (250, 250), (250, 250)), ()),
    ("gemm_f32_mfma_1024x256x1024", "matmul", "float32", ((1024, 1024), (1024, 256), (256, 1024)), ()),
    ("gemm_f32_ragged_1000x1000x520", "matmul", "float32", ((1000, 1000), (1000, 520), (520, 1000)), ()),
    ("conv_f16_c3", "conv2d", "float16", ((32, 64, 56, 56), (32, 64, 56, 56), (64, 64, 3, 3)), (1, 1, 1, 1, 1, 1, 1, 1)),
    ("conv_bf16_3x64x20x40", "conv2d", "bfloat16", ((3, 64, 20, 40), (3, 64, 20, 40), (64, 64, 3, 3)),
     (1, 1, 1, 1, 1, 1, 1, 1)),
    ("conv_f16_2x64x12x24", "conv2d", "float16", ((2, 64, 12, 24), (2, 64, 12, 24), (64, 64, 3, 3)),
     (1, 1, 1, 1, 1, 1, 1, 1)),
    ("conv_f16_igemm_2x64x50x50_s2", "conv2d", "float16", ((2, 64, 25, 25), (2, 64, 50, 50), (64, 64, 3, 3)),
     (2, 2, 1, 1, 1, 1, 1, 1)),
    ("conv_f32_igemm_1x40x19x23_f96", "conv2d", "float32", ((1, 96, 18, 12), (1, 40, 19, 23), (96, 40, 3, 3)),
     (1, 2, 2, 1, 2, 1, 0, 3)),
    ("conv_f16_rowvec_2x128x28x28", "conv2d", "float16", ((2, 128, 28, 28), (2, 128, 28, 28), (128, 128, 3, 3)),
     (1, 1, 1, 1, 1, 1, 1, 1)),
    ("conv_bf16_rowvec_1x1_2x64x16x32_f96", "conv2d", "bfloat16", ((2, 96, 16, 32), (2, 64, 16, 32), (96, 64, 1, 1)),
     (1, 1, 1, 1, 0, 0, 0, 0)),
    ("conv_f16_rowvec_s2_2x64x56x56", "conv2d", "float16", ((2, 128, 28, 28), (2, 64, 56, 56), (128, 64, 3, 3)),
     (2, 2, 1, 1, 1, 1, 1, 1)),
    ("conv_f32_rowvec_2x64x28x28_f96", "conv2d", "float32", ((2, 96, 28, 28), (2, 64, 28, 28), (96, 64, 3, 3)),
     (1, 1, 1, 1, 1, 1, 1, 1)),
    ("fa_bf16_c4", "flash_attention", "bfloat16", ((4, 32, 2048, 128),) * 4, (128, 64, 0.088388, 0)),
    ("fa_bf16_causal_1x4x4096x128", "flash_attention", "bfloat16", ((1, 4, 4096, 128),) * 4, (128, 64, 0.088388, 1)),
    ("fa_f16_causal_1x2x1000x64", "flash_attention", "float16", ((1, 2, 1000, 64),) * 4, (128, 64, 0.125, 1)),
    ("fa_bf16_2x3x130x128", "flash_attention", "bfloat16", ((2, 3, 130, 128),) * 4, (128, 64, 0.088388, 0)),
    ("fa_f32_causal_1x2x700x128", "flash_attention", "float32", ((1, 2, 700, 128),) * 4, (64, 64, 0.088388, 1)),
    ("fa_f32_2x1x130x64", "flash_attention", "float32", ((2, 1, 130, 64),) * 4, (64, 64, 0.125, 0)),
)


def _slots(family: str, operands: list, scalars: tuple) -> list:
    if family == "flash_attention":
        return [*operands, *scalars]
    return [*operands, None, *scalars]


def modelled(case) -> dict[str, int]:
    name, family, dtype, shapes, scalars = case
    return native.cost(family, _slots(family, [native.TensorSpec(s, dtype) for s in shapes], scalars))


def prepare(case, device: str = "cuda"):
    """(entry name, slot args) of a case, with its tensors made on the host and copied."""

    import torch

    name, family, dtype, shapes, scalars = case
    dt = getattr(torch, dtype)
    gen = torch.Generator().manual_seed(7)  # host-side values: the only device work is the copy
    tensors = [torch.randn(s, generator=gen, dtype=torch.float32).to(dt).to(device) for s in shapes]
    torch.cuda.synchronize()
    entry = {"matmul": "kg_gfx950_matmul_entry", "conv2d": "kg_gfx950_conv2d_entry",
             "flash_attention": "kg_gfx950_flash_attention_entry"}[family]
    return entry, _slots(family, tensors, scalars)


def run(case, device: str = "cuda") -> None:
    entry, args = prepare(case, device)
    native.call_entry(entry, args)


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--model-only", action="store_true", help="print the modelled costs without a GPU")
    opts = parser.parse_args(argv)
    for case in CASES:
        line = {"case": case[0], **modelled(case)}
        if not opts.model_only:
            run(case)
            line["ran"] = True
        print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
