"""asa_forward_noalloc (the forward whose workspace is the library's own
device array) against asa_forward, through the C ABI: two calls in a row,
the second on a smaller problem, every output and state buffer bit for bit.
No reference counterpart (the reference allocates inside the extension)."""
import pytest
import torch

from tests._util import causal_idx, make_inputs

pytestmark = pytest.mark.gpu

# (B, H, N, d, dtype, k_keep, alpha, scale): the second is smaller, so the
# shared array holds stale data from the first call when the second runs
CASES = [
    (2, 8, 1536, 64, torch.bfloat16, 32, 1.5, 0.125),
    (1, 3, 300, 64, torch.bfloat16, 8, 1.5, 0.125),
]


def _forward(noalloc, Q, K, V, idx, k, alpha, scale):
    from splash_attention import ops

    out, st = ops.splash_forward(Q, K, V, idx, idx, alpha, k, scale, with_topk=True,
                                 with_support=True, noalloc=noalloc)
    torch.cuda.synchronize()
    return out, st


def test_noalloc_forward_matches_forward_twice(dev):
    for B, H, N, d, dtype, k, alpha, scale in CASES:
        print(f"[noalloc] B={B} H={H} N={N} d={d} {dtype} k={k}", flush=True)
        Q, K, V, _ = (t.to(dev) for t in make_inputs(B, H, N, N, d, seed=3, dtype=dtype))
        idx = causal_idx(B * H, N).to(dev)
        want_out, want = _forward(False, Q, K, V, idx, k, alpha, scale)
        got_out, got = _forward(True, Q, K, V, idx, k, alpha, scale)
        assert torch.equal(got_out.view(torch.int16), want_out.view(torch.int16))
        for name in ("taus", "norms", "mask", "q_ptr", "q_list", "k_ptr", "k_list",
                     "topk_idx", "topk_val", "status"):
            a, b = getattr(got, name), getattr(want, name)
            if a.dtype.is_floating_point:
                a, b = a.view(torch.int32), b.view(torch.int32)
            assert torch.equal(a, b), name
        # support masks exist for the active tiles only (q_list positions
        # below q_ptr[bh, nQB]); the rest of the buffer is never written
        for bh in range(B * H):
            n = int(want.q_ptr[bh, -1])
            assert torch.equal(got.sup_mask[bh, :n], want.sup_mask[bh, :n]), f"sup_mask {bh}"
        got.check_status()


def test_noalloc_rejects_problems_above_its_workspace(dev):
    from splash_attention import _lib, ops

    # 64 * 32768 rows x k 128 x 4 bytes of sorted top-k values: 1 GiB
    p = ops.make_problem(4, 16, 32768, 32768, 64, torch.bfloat16, 1.5, 128, 0.125)
    assert _lib.query_sizes(p).workspace > _lib.NOALLOC_WORKSPACE_BYTES
    lib = _lib.load()
    rc = lib.asa_forward_noalloc(p, None, None, None, None, None, None, None, None)
    assert rc == _lib.ASA_ERR_UNSUPPORTED
    assert "asa_forward_noalloc holds" in lib.asa_last_error().decode()


def test_noalloc_forward_replays_in_a_hip_graph(dev):
    """The stated use of asa_forward_noalloc: capture it in a HIP graph
    (torch.cuda.CUDAGraph) after a first call outside capture (which looks
    up the array's address), then replay it three times, each on new inputs
    copied into the captured buffers and with eager work between replays;
    every replay equals an eager asa_forward call on the same inputs bit for
    bit.  The forward records no hipMemsetAsync (its first kernel clears
    what must start at zero)."""
    from splash_attention import ops

    B, H, N, d, k, alpha, scale = 1, 4, 512, 64, 16, 1.5, 0.125
    print(f"[noalloc] graph capture B={B} H={H} N={N} d={d} bf16 k={k}", flush=True)
    Q, K, V, _ = (t.to(dev) for t in make_inputs(B, H, N, N, d, seed=5, dtype=torch.bfloat16))
    idx = causal_idx(B * H, N).to(dev)
    sQ, sK, sV = Q.clone(), K.clone(), V.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.splash_forward(sQ, sK, sV, idx, idx, alpha, k, scale, with_topk=True, noalloc=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout, gst = ops.splash_forward(sQ, sK, sV, idx, idx, alpha, k, scale, with_topk=True,
                                       noalloc=True)
    torch.cuda.synchronize()
    for rep in range(3):
        nQ, nK, nV, _ = make_inputs(B, H, N, N, d, seed=40 + rep, dtype=torch.bfloat16)
        sQ.copy_(nQ)
        sK.copy_(nK)
        sV.copy_(nV)
        graph.replay()
        torch.cuda.synchronize()
        want_out, want = ops.splash_forward(sQ, sK, sV, idx, idx, alpha, k, scale,
                                            with_topk=True)
        torch.cuda.synchronize()
        assert torch.equal(gout.view(torch.int16), want_out.view(torch.int16)), f"replay {rep}"
        for name in ("taus", "norms", "mask", "q_ptr", "q_list", "k_ptr", "k_list",
                     "topk_idx", "topk_val", "status"):
            a, b = getattr(gst, name), getattr(want, name)
            if a.dtype.is_floating_point:
                a, b = a.view(torch.int32), b.view(torch.int32)
            assert torch.equal(a, b), f"replay {rep}: {name}"
        for bh in range(B * H):
            n = int(want.q_ptr[bh, -1])
            assert torch.equal(gst.sup_mask[bh, :n], want.sup_mask[bh, :n]), f"sup_mask {bh}"
    del graph
