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
