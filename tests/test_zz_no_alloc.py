"""GPU test of qe_moe_dispatch_noalloc (no allocation, scratch in a static
device array) against qe_moe_dispatch of a context, called through the C ABI:
two calls in a row, the second smaller, each bit-exact (off and pairs); and the
same call captured into a HIP graph (through torch.cuda.graph) and replayed on
new ids, with eager work between the replays."""
import numpy as np
import pytest

import oracle as O
import qe_moe

pytestmark = pytest.mark.gpu


def skewed_ids(rng, T):
    # every expert appears, a few are heavy (Zipf-like), no expert twice per token
    p = 1.0 / np.arange(1, 257) ** 1.1
    p /= p.sum()
    perm = rng.permutation(256)
    return np.stack([perm[rng.choice(256, 8, replace=False, p=p)] for _ in range(T)]).astype(np.int32)


def test_dispatch_noalloc_matches_context_dispatch(torch_cuda):
    torch = torch_cuda
    tmax = qe_moe.QE_MOE_DISPATCH_NOALLOC_T_MAX
    m = qe_moe.MoE(n_layers=1, t_max=tmax)
    try:
        rng = np.random.default_rng(31)
        off = torch.empty(257, dtype=torch.int32, device="cuda")
        for T in (tmax, 777):  # the largest size, then a smaller call over the same static scratch
            print(f"dispatch_noalloc T={T}", flush=True)
            ids = skewed_ids(rng, T)
            ids_d = torch.from_numpy(ids).cuda()
            pairs = torch.full((T * 8,), -1, dtype=torch.int32, device="cuda")
            off.fill_(-1)
            qe_moe.dispatch_noalloc(ids_d, T, off, pairs)
            m.dispatch(ids_d, T)  # the context entry point
            r = m.routing(T)
            torch.cuda.synchronize()
            assert np.array_equal(off.cpu().numpy(), r["off"]) and np.array_equal(pairs.cpu().numpy(), r["pairs"])
            o_off, o_pairs = O.dispatch(ids)
            assert np.array_equal(r["off"], o_off) and np.array_equal(r["pairs"], o_pairs)
        with pytest.raises(qe_moe.QeError) as e:
            qe_moe.dispatch_noalloc(ids_d, tmax + 1, off, pairs)
        assert e.value.code == qe_moe.QE_ERR_ARG
    finally:
        m.close()


def test_dispatch_noalloc_under_graph_capture(torch_cuda):
    # The context created first has looked the static scratch up, so the very
    # first no-allocation call can be the captured one.  The graph holds the two
    # dispatch kernels (no memset node); every replay reads the ids buffer anew.
    torch = torch_cuda
    T = 3000
    m = qe_moe.MoE(n_layers=1, t_max=T)
    try:
        rng = np.random.default_rng(32)
        ids_d = torch.from_numpy(skewed_ids(rng, T)).cuda()
        off = torch.full((257,), -1, dtype=torch.int32, device="cuda")
        pairs = torch.full((T * 8,), -1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        print("dispatch_noalloc: capture", flush=True)
        with torch.cuda.graph(g):
            qe_moe.dispatch_noalloc(ids_d, T, off, pairs, stream=torch.cuda.current_stream())
        for rep in range(4):
            ids = skewed_ids(rng, T)
            ids_d.copy_(torch.from_numpy(ids))
            off.fill_(-1)
            pairs.fill_(-1)
            print(f"dispatch_noalloc: replay {rep}", flush=True)
            g.replay()
            torch.cuda.synchronize()
            m.dispatch(ids_d, T)
            r = m.routing(T)
            assert np.array_equal(off.cpu().numpy(), r["off"]) and np.array_equal(pairs.cpu().numpy(), r["pairs"]), rep
            o_off, o_pairs = O.dispatch(ids)
            assert np.array_equal(r["off"], o_off) and np.array_equal(r["pairs"], o_pairs)
    finally:
        m.close()
