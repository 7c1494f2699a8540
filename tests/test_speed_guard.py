"""Speed guards for the register top-k path (C1's single row, C2's chunks).

A register row whose selection bound comes out wrong is not an error: the
row is sampled again by the general paths, and the tokens stay exact.  Only
the time shows it (about twice the time for C2 and C1).  These tests bound
the time of one C2 batch and of one C1 row on the device, with room for box
to box variation (the bounds are about 1.5 times the measured times), so
that such a silent fallback fails here instead of passing the parity tests.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _median_us(torch, call, reps=30, rounds=5):
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(5):
        call(st)
    torch.cuda.synchronize()
    ts = []
    for _ in range(rounds):
        e0.record(st)
        for _ in range(reps):
            call(st)
        e1.record(st)
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / reps)
    return float(np.median(ts))


def test_c2_batch_time(gpu, torch):
    import workloads
    w = workloads.make("c2")
    c = workloads.CONFIGS["c2"]
    B, V = w["B"], w["V"]
    _say("c2 speed guard: B=%d V=%d" % (B, V))
    s = gpu.Sampler(c["T"], c["k"], c["p"], c["rep"], seed=42)
    s.reserve(B, V)
    lg = torch.from_numpy(w["logits"]).cuda()
    rec = torch.from_numpy(w["recent"].view(np.int32)).cuda()
    u = torch.from_numpy(w["u"]).cuda()
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    us = _median_us(torch, lambda st: s.sample_batch(lg, tok, recent=rec, u=u, stream=st))
    _say("c2: %.1f us per batch" % us)
    assert us < 30.0, "C2 batch took %.1f us (about 21 expected): rows fell back to the general paths?" % us


def test_c1_row_time(gpu, torch):
    import workloads
    w = workloads.make("c1", steps=1)
    _say("c1 speed guard: V=%d" % w["V"])
    lg = torch.from_numpy(w["logits"]).cuda()
    win = torch.from_numpy(w["init_recent"].view(np.int32)).cuda().reshape(1, w["W"])
    u = torch.zeros(1, dtype=torch.float32, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(w["T"], w["k"], w["p"], w["rep"], seed=w["seed"])
    us = _median_us(torch, lambda st: s.sample_batch(lg, tok, recent=win, u=u, stream=st), reps=100)
    _say("c1: %.1f us per row" % us)
    assert us < 21.0, "C1 row took %.1f us (about 14 expected): the row fell back to the general path?" % us
