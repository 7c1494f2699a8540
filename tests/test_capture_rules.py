"""Stream and graph rules of the batched entry (include/gs_sampler.h):
- under HIP graph capture a call that would take its draws from the
  sampler's host LCG (d_u == NULL, T > 0) is refused with
  GS_ERR_UNSUPPORTED (a graph would replay the draws frozen at capture);
- once a call has been captured, a later call that needs bigger buffers
  leaves the captured graph's buffers alive: the graph still replays
  correctly;
- the Python sample() on device logits waits for torch's current stream,
  which may still be writing them."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_capture_without_draws_rejected(gpu, torch):
    V, B = 32000, 4
    d_lg = torch.randn((B, V), device="cuda")
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    u = torch.rand(B, device="cuda")
    s = gpu.Sampler(0.7, 40, 0.9, 1.0, seed=1)
    s.reserve(B, V)
    s.sample_batch(d_lg, tok, u=u)                      # warm-up outside the capture
    torch.cuda.synchronize()
    _say("capture with d_u == NULL")
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(g):
        tok.add_(0)
        try:
            s.sample_batch(d_lg, tok)                   # host LCG draws: refused
        except gpu.SamplerError as e:
            err = e.code
        s.sample_batch(d_lg, tok, u=u)                  # device draws: captured
    assert err == gpu.GS_ERR_UNSUPPORTED
    g.replay()
    torch.cuda.synchronize()


def test_grow_after_capture_keeps_graph_buffers(gpu, torch, oracle):
    """A graph of a small full-vocabulary batch, then an eager call on a
    larger batch (the scratch grows), then the graph again: its rows must
    still be sampled exactly."""
    import workloads
    V = 50000
    rng = np.random.default_rng(9)
    lg = (rng.standard_normal((2, V)) * 2).astype(np.float32)
    u = np.array([0.3, 0.97], np.float32)
    params = workloads.params_rows([(1.0, 0, 0.95, 1.0)] * 2)
    want = oracle.sample_batch(lg, params, u)
    d_lg = torch.from_numpy(lg).cuda()
    d_u = torch.from_numpy(u).cuda()
    tok = torch.zeros(2, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(1.0, 0, 0.95, 1.0, seed=1)
    s.reserve(2, V)
    s.sample_batch(d_lg, tok, u=d_u)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s.sample_batch(d_lg, tok, u=d_u)
    _say("grow: eager batch of 64 rows after the capture")
    big = torch.randn((64, V), device="cuda")
    tbig = torch.zeros(64, dtype=torch.int32, device="cuda")
    s.sample_batch(big, tbig, u=torch.rand(64, device="cuda"))
    torch.cuda.synchronize()
    for _ in range(3):
        tok.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(tok.cpu().numpy().astype(np.int64), want)


def test_python_sample_waits_for_torch_stream(gpu, torch, oracle):
    """The logits are written by a torch kernel queued behind a long chain
    of work on torch's stream; sample() must see the written values."""
    V = 32000
    rng = np.random.default_rng(4)
    host = (rng.standard_normal(V) * 3).astype(np.float32)
    host[rng.integers(0, V, 5)] += 10.0
    src = torch.from_numpy(host).cuda()
    d = torch.zeros(V, device="cuda")
    a = torch.randn((4096, 4096), device="cuda")
    torch.cuda.synchronize()
    for _ in range(8):
        a = a @ a * 1e-2                                # keeps torch's stream busy
    d.copy_(src)                                        # the logits, queued last
    gpu.set_seed(123)
    tok = gpu.sample(d, 0.7, 40, 0.9, 1.1, ())
    torch.cuda.synchronize()
    oracle.set_seed(123)
    want = oracle.sample(host, 0.7, 40, 0.9, 1.1, ())
    assert tok == want
