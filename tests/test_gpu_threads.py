"""The launch mode is per host thread (kg_gfx950_set_launch_mode).

ctypes releases the GIL during a foreign call, so two Python threads can be inside the
library at once. One thread runs synchronous calls (the reference's execute() contract,
kernel_gen/execute_engine/compiler.py:286-291: the call returns after the kernel ran);
the other enqueues on its own stream. Each must see its own mode: the synchronous
thread's results are complete when its call returns, and the stream thread's results are
complete after its stream synchronizes. Both are checked against the oracle.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest

from kernelcode_generate_amd import native
from tests.gpu_util import assert_h16_close, round_to, to_numpy

pytestmark = pytest.mark.gpu


def test_sync_and_stream_threads(device, oracle_mod):
    import torch

    rng = np.random.default_rng(99)
    m, k, n = 512, 1024, 512
    lt, lhs = round_to(rng.standard_normal((m, k), dtype=np.float32) * 0.05, torch.bfloat16)
    rt, rhs = round_to(rng.standard_normal((k, n), dtype=np.float32) * 0.05, torch.bfloat16)
    a, b = lt.to(device), rt.to(device)
    ref = oracle_mod.matmul_demo(lhs, rhs, None, (64, 64, 64))
    torch.cuda.synchronize()
    rounds = 20
    errors: list[BaseException] = []
    results: dict[str, list] = {"sync": [], "stream": []}
    start = threading.Barrier(2)

    def sync_worker():
        try:
            native.set_launch_mode(True, None)
            start.wait()
            for _ in range(rounds):
                out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
                torch.cuda.synchronize()
                native.matmul(out, a, b, None)
                # synchronous: the result is complete when the call returns; copy it on a
                # side stream that never waits on the default stream's later work
                results["sync"].append(out.clone())
        except BaseException as exc:  # noqa: BLE001 - reported by the main thread
            errors.append(exc)

    def stream_worker():
        try:
            stream = torch.cuda.Stream()
            native.set_launch_mode(False, stream.cuda_stream)
            start.wait()
            outs = []
            with torch.cuda.stream(stream):
                for _ in range(rounds):
                    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
                    native.matmul(out, a, b, None)
                    outs.append(out)
            stream.synchronize()
            results["stream"] = outs
            native.set_launch_mode(True, None)
        except BaseException as exc:  # noqa: BLE001
            errors.append(exc)

    print("[threads] one synchronous and one stream thread, 20 bf16 matmuls each", flush=True)
    threads = [threading.Thread(target=sync_worker), threading.Thread(target=stream_worker)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    assert len(results["sync"]) == rounds and len(results["stream"]) == rounds
    first = results["sync"][0]
    assert_h16_close(to_numpy(first), ref, what="sync thread")
    for name in ("sync", "stream"):
        for i, out in enumerate(results[name]):
            assert torch.equal(out, first), f"{name} round {i} differs"


def test_split_k_threads_on_one_stream(device, oracle_mod):
    """Two synchronous threads on the one default stream, both running split-K matmuls
    (two kernels per call: fp32 partials in the per-stream workspace, then their ordered
    reduction) of different sizes, so the workspace is also replaced while the other thread
    uses it. Each call must hold the workspace from its partials through its reduction:
    every result equals the single-threaded one bit for bit (the split is deterministic)."""

    import torch

    rng = np.random.default_rng(7)
    shapes = ((16, 4096, 4096), (64, 1024, 8192))  # 16 and 4 output tiles: 16- and 32-way K splits
    operands, expected = [], []
    native.set_launch_mode(True, None)
    for m, n, k in shapes:
        a = round_to(rng.standard_normal((m, k), dtype=np.float32) * 0.05, torch.bfloat16)[0].to(device)
        b = round_to(rng.standard_normal((k, n), dtype=np.float32) * 0.05, torch.bfloat16)[0].to(device)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
        native.matmul(out, a, b, None)
        operands.append((a, b))
        expected.append(out.clone())
    ref = oracle_mod.matmul_demo(to_numpy(operands[0][0]), to_numpy(operands[0][1]), None, (64, 64, 64))
    assert_h16_close(to_numpy(expected[0]), ref, "split-K 16x4096x4096")
    torch.cuda.synchronize()
    rounds = 30
    errors: list[BaseException] = []
    mismatches: list[tuple[int, int]] = []
    start = threading.Barrier(2)

    def worker(which: int) -> None:
        try:
            native.set_launch_mode(True, None)
            a, b = operands[which]
            m, n, _ = shapes[which]
            start.wait()
            for r in range(rounds):
                out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
                native.matmul(out, a, b, None)
                if not torch.equal(out, expected[which]):
                    mismatches.append((which, r))
        except BaseException as exc:  # noqa: BLE001 - reported by the main thread
            errors.append(exc)

    print("[threads] two synchronous threads on the default stream, split-K matmuls of two sizes", flush=True)
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
    assert not mismatches, mismatches
