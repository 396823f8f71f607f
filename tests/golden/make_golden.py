"""Write the golden fixtures under tests/golden/ (run from the repository root).

The fixtures hold input/expected-output data taken from the reference's own tests:
  - kat_primitives.npz: the known-answer values of test/include/api/test_kernel.py
    (matmul :199-219, reduce_max :221-235, img2col1d/2d :302-364, exp :249-293);
  - cuda_runtime_vectors.npz: the runtime vectors of
    test/cuda/test_cuda_sm89_kernel_demos_runtime.py (matmul arange inputs :515-526,
    conv2d arange/7 inputs with the demo strides/pads :549-565 for the two small cases,
    flash attention default_rng(2026052901) inputs of shape (1,2,4,3) :586-595), with the
    expected outputs computed by the closed forms those tests use (np.matmul,
    pad + einsum conv, max-shifted softmax attention), evaluated in float64.
No reference code is imported or run to make them.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def conv_closed_form(x, w, bias, stride, dilation, padding):
    pt, pb, pl, pr = padding
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (pt, pb), (pl, pr)))
    n, c, h, ww = xp.shape
    f, _, kh, kw = w.shape
    ho = (h - dilation[0] * (kh - 1) - 1) // stride[0] + 1
    wo = (ww - dilation[1] * (kw - 1) - 1) // stride[1] + 1
    out = np.zeros((n, f, ho, wo))
    for r in range(kh):
        for q in range(kw):
            hs, ws = r * dilation[0], q * dilation[1]
            win = xp[:, :, hs : hs + ho * stride[0] : stride[0], ws : ws + wo * stride[1] : stride[1]]
            out += np.einsum("nchw,fc->nfhw", win, w[:, :, r, q].astype(np.float64))
    if bias is not None:
        out += bias.astype(np.float64)[None, :, None, None]
    return out


def attention_closed_form(q, k, v, scale=1.0, causal=False):
    s = np.matmul(q.astype(np.float64), np.swapaxes(k, -1, -2).astype(np.float64)) * scale
    if causal:
        n = s.shape[-1]
        s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return p @ v.astype(np.float64)


def make_kat() -> dict[str, np.ndarray]:
    return {
        "matmul_lhs": np.array([[1, 2], [3, 4]], np.float32),
        "matmul_rhs": np.array([[5, 6], [7, 8]], np.float32),
        "matmul_expected": np.array([[19, 22], [43, 50]], np.float32),
        "matmul_acc_expected": np.array([[38, 44], [86, 100]], np.float32),
        "reduce_input": np.array([[1, 9, 3], [7, 2, 5]], np.float32),
        "reduce_max_expected": np.array([[9], [7]], np.float32),
        "img2col2d_input": np.arange(1, 10, dtype=np.float32).reshape(1, 1, 3, 3),
        "img2col2d_expected": np.array(
            [1, 2, 4, 5, 2, 3, 5, 6, 4, 5, 7, 8, 5, 6, 8, 9], np.float32
        ).reshape(1, 1, 2, 2, 2, 2),
        "exp_input": np.arange(1, 7, dtype=np.float32).reshape(2, 3),
    }


CONV_CASES = (
    # (input shape, weight shape, stride, dilation, padding (top,bottom,left,right))
    ((1, 2, 21, 29), (3, 2, 2, 2), (8, 8), (1, 1), (4, 3, 4, 3)),
    ((1, 2, 4, 5), (3, 2, 2, 2), (1, 1), (1, 1), (1, 1, 1, 1)),
)
BIG_CONV_CASE = ((4, 49, 248, 232), (20, 49, 3, 5), (8, 8), (1, 1), (3, 3, 4, 0))


def make_runtime() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    lhs = np.arange(6, dtype=np.float32).reshape(2, 3)
    rhs = np.arange(12, dtype=np.float32).reshape(3, 4)
    bias = np.arange(4, dtype=np.float32)
    out.update(
        matmul_lhs=lhs,
        matmul_rhs=rhs,
        matmul_bias=bias,
        matmul_absent=(lhs.astype(np.float64) @ rhs).astype(np.float32),
        matmul_present=(lhs.astype(np.float64) @ rhs + bias).astype(np.float32),
    )
    for i, (xs, ws, stride, dil, pad) in enumerate(CONV_CASES):
        x = np.arange(int(np.prod(xs)), dtype=np.float32).reshape(xs)
        w = np.arange(int(np.prod(ws)), dtype=np.float32).reshape(ws) / np.float32(7.0)
        b = np.arange(ws[0], dtype=np.float32)
        out[f"conv{i}_params"] = np.array([*xs, *ws, *stride, *dil, *pad], np.int64)
        out[f"conv{i}_absent"] = conv_closed_form(x, w, None, stride, dil, pad).astype(np.float32)
        out[f"conv{i}_present"] = conv_closed_form(x, w, b, stride, dil, pad).astype(np.float32)
    xs, ws, stride, dil, pad = BIG_CONV_CASE
    out["conv_big_params"] = np.array([*xs, *ws, *stride, *dil, *pad], np.int64)
    rng = np.random.default_rng(2026052901)
    q = rng.normal(size=(1, 2, 4, 3)).astype(np.float32)
    k = rng.normal(size=(1, 2, 4, 3)).astype(np.float32)
    v = rng.normal(size=(1, 2, 4, 3)).astype(np.float32)
    out.update(fa_q=q, fa_k=k, fa_v=v, fa_expected=attention_closed_form(q, k, v).astype(np.float32))
    return out


def main() -> None:
    np.savez_compressed(HERE / "kat_primitives.npz", **make_kat())
    np.savez_compressed(HERE / "cuda_runtime_vectors.npz", **make_runtime())


if __name__ == "__main__":
    main()
