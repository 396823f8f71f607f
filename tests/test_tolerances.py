"""CPU checks of the 16-bit attention bar (tests/gpu_util.attention_h16_tolerance): the
rounding the kernels' design adds -- P rounded to the 16-bit format before P V, the row
sum over the same rounded P -- simulated in float64 stays inside it, and a planted error
of 5 % of O does not."""

from __future__ import annotations

import numpy as np
import pytest

from tests.gpu_util import assert_within, attention_h16_tolerance
from tests.ir_interp import bf16_round


def _rounded_p_attention(q, k, v, scale, causal, dtype_name):
    s = scale * (q @ np.swapaxes(k, -1, -2))
    if causal:
        s = np.where(np.tril(np.ones(s.shape[-2:], bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    if dtype_name == "bfloat16":
        p16 = bf16_round(p.astype(np.float32)).astype(np.float64)
    else:
        p16 = p.astype(np.float16).astype(np.float64)
    return (p16 @ v) / p16.sum(-1, keepdims=True)


@pytest.mark.parametrize("seq,causal,dtype_name", [(512, False, "bfloat16"), (512, True, "bfloat16"),
                                                    (1024, True, "float16"), (2048, False, "bfloat16")])
def test_bar_holds_the_p_rounding_and_rejects_a_5_percent_error(seq, causal, dtype_name):
    rng = np.random.default_rng(seq + causal)
    shape = (1, 2, seq, 128)
    q, k, v = (rng.standard_normal(shape) for _ in range(3))
    scale = 1.0 / np.sqrt(128)
    bar = attention_h16_tolerance(q, k, v, scale, causal, dtype_name)
    s = scale * (q @ np.swapaxes(k, -1, -2))
    if causal:
        s = np.where(np.tril(np.ones(s.shape[-2:], bool)), s, -np.inf)
    w = np.exp(s - s.max(-1, keepdims=True))
    o = (w / w.sum(-1, keepdims=True)) @ v
    assert_within(_rounded_p_attention(q, k, v, scale, causal, dtype_name), o, bar, "rounded-P simulation")
    with pytest.raises(AssertionError):
        assert_within(o * 1.05, o, bar, "5 % error")
    # a systematic 5 % error shows on a large share of the elements, not on a few outliers
    caught = np.abs(0.05 * o) > bar
    assert caught.mean() > 0.2, caught.mean()
