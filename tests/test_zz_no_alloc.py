"""asa_forward_noalloc (the forward whose workspace is the library's own
device array) against asa_forward, through the C ABI: two calls in a row,
the second on a smaller problem, and a sequence of sixteen drawn problems,
every output and state buffer bit for bit; its size rejection; and the call
captured in a HIP graph.
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


def test_noalloc_random_sequence_matches_forward(dev):
    """Sixteen drawn problems in a row through asa_forward_noalloc, each
    against asa_forward bit for bit (out and every state buffer): dtypes,
    ragged NQ != NK, head dimensions, k, 64- or 32-row mask blocks, both tau
    modes, causal, non-causal or random positions.  The library's array keeps
    the previous call's bytes, of another size and layout, every time."""
    import random

    from splash_attention import ops

    rng = random.Random(7)
    for i in range(16):
        dt = rng.choice([torch.float32, torch.bfloat16, torch.float16])
        step = 4 if dt == torch.float32 else 8
        B, H = rng.choice([1, 2]), rng.choice([1, 2, 3])
        NQ, NK = rng.choice([1, 65, 300, 777, 1024]), rng.choice([1, 64, 200, 640, 1100])
        d = rng.choice([64, 128, rng.randrange(step, 129, step)])
        k, bm = rng.choice([2, 8, 32, 64]), rng.choice([64, 32])
        tau_mode = "exact" if bm == 64 and rng.random() < 0.4 else "reference"
        kind = rng.choice(["causal", "noncausal", "random"])
        seed = rng.randrange(10 ** 6)
        print(f"[noalloc] draw {i}: {str(dt)[6:]} B{B} H{H} NQ{NQ} NK{NK} d{d} k{k} "
              f"block_m {bm} {tau_mode} {kind}", flush=True)
        g = torch.Generator().manual_seed(seed)
        Q = torch.randn(B, H, NQ, d, generator=g).to(dt).to(dev)
        K = torch.randn(B, H, NK, d, generator=g).to(dt).to(dev)
        V = torch.randn(B, H, NK, d, generator=g).to(dt).to(dev)
        if kind == "random":
            qi = torch.randint(0, NK + 3, (B * H, NQ), generator=g).to(torch.int32)
            ki = torch.randint(0, NK + 3, (B * H, NK), generator=g).to(torch.int32)
        else:
            ki = torch.arange(NK, dtype=torch.int32).expand(B * H, NK).contiguous()
            last = NK - 1 if kind == "noncausal" else None
            qi = (torch.full((B * H, NQ), last, dtype=torch.int32) if last is not None else
                  (torch.arange(NQ, dtype=torch.int32) + (NK - NQ)).expand(B * H, NQ).contiguous())
        q, kk, v, qi, ki = ops.check_inputs(Q, K, V, qi.to(dev), ki.to(dev))
        res = []
        for noalloc in (True, False):
            out, st = ops.splash_forward(q, kk, v, qi, ki, 1.5, k, 0.125, with_topk=True,
                                         tau_mode=tau_mode, noalloc=noalloc, block_m=bm)
            torch.cuda.synchronize()
            res.append((out, st))
        (got_out, got), (want_out, want) = res
        assert torch.equal(got_out.view(torch.uint8), want_out.view(torch.uint8)), f"draw {i}: out"
        for name in ("taus", "norms", "mask", "q_ptr", "q_list", "k_ptr", "k_list",
                     "topk_idx", "topk_val", "status"):
            a, b = getattr(got, name), getattr(want, name)
            if a.dtype.is_floating_point:
                a, b = a.view(torch.int32), b.view(torch.int32)
            assert torch.equal(a, b), f"draw {i}: {name}"
        # support masks of the active 64-row tiles (the kernels' tiles: with
        # 32-row mask blocks, the union of each pair of mask rows)
        m = want.mask.reshape(B * H, -1, want.mask.shape[-1]) != 0
        if bm == 32:
            if m.shape[1] % 2:
                m = torch.cat([m, torch.zeros_like(m[:, :1])], 1)
            m = m.reshape(B * H, -1, 2, m.shape[-1]).any(2)
        for bh in range(B * H):
            n = int(m[bh].sum())
            assert torch.equal(got.sup_mask[bh, :n], want.sup_mask[bh, :n]), f"draw {i}: sup {bh}"
