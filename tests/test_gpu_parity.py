"""GPU parity of the HIP MoE block against the CPU oracle (needs an MI355X).

Bar (north star): routing ids, the dispatch permutation and offsets bit-exact;
router logits bit-exact (canonical order shared with the oracle); layer
outputs within 1e-3 relative L2, and the shared-expert term separately within
1e-3 (it is ~1e-5 of the output norm, so the total does not constrain it).
Weights are within 2e-6 (the GPU and the oracle use their own expf).
"""
import numpy as np
import pytest

import oracle as O
import qe_moe

pytestmark = pytest.mark.gpu
SEED = 0xC0FFEE
TOL = 1e-3


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b.astype(np.float64)), 1e-30))


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def ctx(torch_cuda):
    m = qe_moe.MoE(n_layers=2, t_max=8192)
    yield m
    m.close()


_layers = {}


def host_layer(layer, bias_s):
    key = (layer, bias_s)
    if key not in _layers:
        bias = None if bias_s is None else O.gen_zipf_bias(SEED, layer, bias_s)
        _layers[key] = O.SynthLayer(SEED, layer, bias=bias)
    return _layers[key]


def run_gpu(torch, ctx, layer, bias_s, x_host, norm=False):
    L = host_layer(layer, bias_s)
    ctx.synth_layer(layer, SEED, L.bias)
    x = torch.from_numpy(x_host).cuda()
    y = torch.empty_like(x)
    T = x_host.shape[0]
    if norm:
        ctx.forward(layer, x, y, T)
    else:
        ctx.forward_normed(layer, x, y, T)
    torch.cuda.synchronize()
    r = ctx.routing(T)
    r["logits"] = ctx.logits(T)
    r["out"] = y.cpu().numpy()
    return L, r


def check_layer(L, g, x, norm=False, sample=None):
    T = x.shape[0]
    ref_in = x if sample is None else x[sample]
    o = O.moe_layer(L, ref_in, norm=norm, residual=norm)
    gi = slice(None) if sample is None else sample
    assert np.array_equal(g["logits"][gi].view(np.uint32), o["logits"].view(np.uint32)), "router logits differ"
    assert np.array_equal(g["ids"][gi], o["ids"]), "routing ids differ"
    assert np.abs(g["wts"][gi] - o["wts"]).max() <= 2e-6
    assert np.abs(g["shg"][gi] - o["shg"]).max() <= 2e-6
    if sample is None:
        assert np.array_equal(g["off"], o["off"]) and np.array_equal(g["pairs"], o["pairs"]), "dispatch differs"
    e_out = rel_l2(g["out"][gi], o["out"])
    e_sd = rel_l2(g["sd"][gi], o["sd"])
    say(f"  T={T} out rel-L2 {e_out:.2e}  shared rel-L2 {e_sd:.2e}")
    assert e_out <= TOL and e_sd <= TOL
    return o


def test_synthetic_bytes_match_host_generator(ctx, torch_cuda):
    torch = torch_cuda
    say("synth bytes: layer 0")
    ctx.synth_layer(0, SEED, None)
    torch.cuda.synchronize()
    base = ctx.arena_ptr(0)
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    for e in (0, 1, 137, 255):
        buf = np.empty(O.EXPERT_BYTES, np.uint8)
        assert hip.hipMemcpy(ctypes.c_void_p(buf.ctypes.data), ctypes.c_void_p(base + e * O.EXPERT_BYTES),
                             ctypes.c_size_t(O.EXPERT_BYTES), 2) == 0
        assert np.array_equal(buf, O.gen_expert(SEED, 0, e)), e
    x = torch.empty(3 * 2048, device="cuda")
    qe_moe.synth_x(SEED, 5, x, x.numel())
    assert np.array_equal(x.cpu().numpy().reshape(3, 2048), O.gen_x(SEED, 5, 3))


@pytest.mark.parametrize("T", [1, 2, 5])
def test_decode_small_T_no_bias(ctx, torch_cuda, T):
    say(f"decode T={T} no bias")
    x = O.gen_x(SEED, 100 + T, T)
    L, g = run_gpu(torch_cuda, ctx, 0, None, x)
    check_layer(L, g, x)


def test_cfg0_decode_B1(ctx, torch_cuda):
    say("config 0: B=1")
    x = O.gen_x(SEED, 0, 1)
    L, g = run_gpu(torch_cuda, ctx, 0, None, x)
    check_layer(L, g, x)


def test_cfg1_decode_B8_zipf(ctx, torch_cuda):
    say("config 1: B=8, Zipf s=1.0 bias")
    x = O.gen_x(SEED, 1, 8)
    L, g = run_gpu(torch_cuda, ctx, 1, 1.0, x)
    check_layer(L, g, x)


@pytest.mark.parametrize("T", [1, 8, 9, 16])
def test_forward_with_norm_and_residual(ctx, torch_cuda, T):
    say(f"forward (norm + residual) T={T}")
    x = O.gen_x(SEED, 200 + T, T)
    L, g = run_gpu(torch_cuda, ctx, 1, 1.0, x, norm=True)
    check_layer(L, g, x, norm=True)


@pytest.mark.parametrize("T", [1, 5, 9, 100])
def test_forward_with_exit_norm(ctx, torch_cuda, T):
    # qe_moe_forward_norm: the layer output as qe_moe_forward, plus the next
    # block's input norm of it; the norm is the canonical one, so it matches the
    # oracle's RMSNorm of the GPU's own output bit for bit.
    torch = torch_cuda
    say(f"forward + exit norm T={T}")
    x = O.gen_x(SEED, 500 + T, T)
    L = host_layer(1, 1.0)
    ctx.synth_layer(1, SEED, L.bias)
    w = (1.0 + 0.25 * O.gen_x(SEED, 600, 1)[0]).astype(np.float32)  # a non-trivial norm weight
    xt = torch.from_numpy(x).cuda()
    wt = torch.from_numpy(w).cuda()
    y = torch.empty_like(xt)
    xn = torch.full_like(xt, float("nan"))
    ctx.forward_norm(1, xt, y, T, wt, xn)
    torch.cuda.synchronize()
    g = ctx.routing(T)
    g["logits"] = ctx.logits(T)
    g["out"] = y.cpu().numpy()
    check_layer(L, g, x, norm=True)
    ref = O.rmsnorm(g["out"], w)
    assert np.array_equal(xn.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    # the plain forward gives the same layer output
    y2 = torch.empty_like(xt)
    ctx.forward(1, xt, y2, T)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    with pytest.raises(qe_moe.QeError):
        ctx.forward_norm(1, xt, y, T, wt, y)


def test_cfg3_prefill_512(ctx, torch_cuda):
    say("config 3: prefill 512, Zipf s=1.0")
    x = O.gen_x(SEED, 3, 512)
    L, g = run_gpu(torch_cuda, ctx, 0, 1.0, x)
    o = check_layer(L, g, x)
    cnt = np.diff(o["off"])
    say(f"  distinct experts {np.count_nonzero(cnt)}, max tokens/expert {cnt.max()}")


def test_cfg4_prefill_8192_skewed(ctx, torch_cuda):
    # every token: logits and ids bit for bit, the dispatch, and the outputs (the
    # oracle's full layer at 8192 tokens takes seconds on the host's cores)
    say("config 4: prefill 8192, Zipf s=1.3 (routing, dispatch and outputs on all tokens)")
    x = O.gen_x(SEED, 4, 8192)
    L, g = run_gpu(torch_cuda, ctx, 1, 1.3, x)
    o = check_layer(L, g, x)
    cnt = np.diff(o["off"])
    say(f"  distinct {np.count_nonzero(cnt)}, max/expert {cnt.max()}, <4 tokens {int(((cnt > 0) & (cnt < 4)).sum())}")


def test_prefill_at_abi_max_T(torch_cuda):
    """T = QE_MOE_T_MAX (65,536 tokens, 524,288 pairs), the largest call the ABI
    accepts, with config 4's Zipf s=1.3 bias: logits, ids, offsets and the
    permutation on every token, outputs on a sample of 4096 tokens spread over
    the call (each token's output depends on its own row only)."""
    torch = torch_cuda
    T = qe_moe.QE_MOE_T_MAX
    m = qe_moe.MoE(n_layers=1, t_max=T)
    try:
        say(f"prefill at the ABI maximum: T={T}, Zipf s=1.3")
        L = O.SynthLayer(SEED, 0, bias=O.gen_zipf_bias(SEED, 0, 1.3))
        m.synth_layer(0, SEED, L.bias)
        x = O.gen_x(SEED, 65, T)
        xd = torch.from_numpy(x).cuda()
        y = torch.empty_like(xd)
        m.forward_normed(0, xd, y, T)
        torch.cuda.synchronize()
        g = m.routing(T)
        g["logits"] = m.logits(T)
        g["out"] = y.cpu().numpy()
        lg = O.router(x, L.router, L.bias)
        assert np.array_equal(g["logits"].view(np.uint32), lg.view(np.uint32)), "router logits differ"
        ids, _, _ = O.topk(lg)
        assert np.array_equal(g["ids"], ids), "routing ids differ"
        off, pairs = O.dispatch(ids)
        assert np.array_equal(g["off"], off) and np.array_equal(g["pairs"], pairs), "dispatch differs"
        sample = np.sort(np.random.default_rng(65).choice(T, 4096, replace=False))
        check_layer(L, g, x, sample=sample)
        cnt = np.diff(off)
        say(f"  distinct {np.count_nonzero(cnt)}, max/expert {cnt.max()}, <4 tokens {int(((cnt > 0) & (cnt < 4)).sum())}")
    finally:
        m.close()


@pytest.mark.parametrize("T,norm", [(33, False), (100, True), (257, False), (2085, True), (4133, False)])
def test_prefill_ragged_T(ctx, torch_cuda, T, norm):
    # T off the 32-token shared-expert tiles and the 64-token router tiles; the
    # context ran larger T before, so the padding rows of the last tiles hold
    # stale activations that must not leak into any output row.  2085 takes the
    # large-T launches (separate router and 64-token shared gate/up tiles) with a
    # last token pair that has one 32-token tile past T (4133: the same with 65
    # token pairs)
    say(f"prefill T={T} (ragged tiles), norm+residual={norm}")
    x = O.gen_x(SEED, 300 + T, T)
    L, g = run_gpu(torch_cuda, ctx, 1, 1.0, x, norm=norm)
    check_layer(L, g, x, norm=norm)


@pytest.mark.parametrize("T", [16, 17, 32, 33, 64, 65, 130, 2064, 2081])
def test_prefill_item_boundaries(ctx, torch_cuda, T):
    # A large bias on 8 experts routes every token to them, so each holds exactly
    # T pairs and the work items take every size class: 16 | 17 (one 16-pair
    # tile | two), 32 | 33 (two tiles | four), 64 | 65 (a full item | plus a
    # one-pair remainder), 130 (two full items and a two-pair remainder).
    # 2064 | 2081: 32 full items and a 16 | 33-pair remainder (the remainder
    # items on the one-matrix gate/up waves | with the full items).
    torch = torch_cuda
    say(f"prefill item boundaries: 8 experts x {T} pairs")
    bias = np.zeros(256, np.float32)
    hot = [3, 40, 77, 128, 129, 200, 254, 255]
    bias[hot] = 50.0
    L = O.SynthLayer(SEED, 0, bias=bias)
    ctx.synth_layer(0, SEED, bias)
    x = O.gen_x(SEED, 400 + T, T)
    xt = torch.from_numpy(x).cuda()
    y = torch.empty_like(xt)
    ctx.forward_normed(0, xt, y, T)
    torch.cuda.synchronize()
    g = ctx.routing(T)
    g["logits"] = ctx.logits(T)
    g["out"] = y.cpu().numpy()
    o = check_layer(L, g, x)
    cnt = np.diff(o["off"])
    assert sorted(np.flatnonzero(cnt).tolist()) == hot and set(cnt[hot].tolist()) == {T}


NEAR_BIAS = {0: 0.0, 1: 1e-6, 16: 2e-6, 32: 3e-6}


def tied_layer(kind, x=None):
    """Layer 1's synthetic weights with a router that forces equal logits (or,
    for "near", logits a few ulps apart; the shared row is turned towards the
    first token of x, so that the group is in that token's top 8)."""
    bias = None
    if kind == "near":
        bias = np.zeros(256, np.float32)
        for e, b in NEAR_BIAS.items():
            bias[e] = b
    L = O.SynthLayer(SEED, 1, bias=bias)
    R = L.router.copy()
    if kind == "zero":  # every logit 0: top-8 is the tie order itself
        R[:] = 0.0
    else:  # experts 0, 1, 16, 32 share one (scaled-up) row: ties between large logits
        R[0] *= 8.0
        if kind == "near" and x is not None and float(np.dot(x[0].astype(np.float64), R[0])) < 0.0:
            R[0] = -R[0]
        R[1] = R[16] = R[32] = R[0]
    L.router = np.ascontiguousarray(R, np.float32)
    return L


@pytest.mark.parametrize("kind", ["zero", "dup", "near"])
@pytest.mark.parametrize("T", [1, 5, 64])
def test_topk_ties_on_gpu(ctx, torch_cuda, kind, T):
    # ties go to the smaller (e % 16, e / 16): all-equal logits select 0, 16, ..., 112.
    # "near": the shared row plus biases of 0, 1, 2, 3 x 1e-6 puts the four experts'
    # logits a few ulps apart (|logit| of a few units has ulps of 2.4e-7 .. 9.5e-7), not
    # equal: the order must follow the values, down to the last bit
    say(f"top-8 ties ({kind} router), T={T}")
    x = O.gen_x(SEED, 400 + T, T)
    L = tied_layer(kind, x)
    ctx.synth_layer(1, SEED, L.bias)
    ctx.set_dense(1, router=L.router)
    xd = torch_cuda.from_numpy(x).cuda()
    y = torch_cuda.empty_like(xd)
    ctx.forward_normed(1, xd, y, T)
    torch_cuda.cuda.synchronize()
    g = ctx.routing(T)
    g["logits"] = ctx.logits(T)
    g["out"] = y.cpu().numpy()
    o = check_layer(L, g, x)
    if kind == "zero":
        assert (o["ids"] == np.arange(0, 128, 16)).all()
    else:
        tied = np.isin(o["ids"], [0, 1, 16, 32]).sum(axis=1)
        say(f"  tokens with the tied group in their top-8: {(tied == 4).sum()} of {T}")
        if kind == "near":
            grp = o["logits"][:, [0, 1, 16, 32]]
            distinct = (np.diff(np.sort(grp, axis=1), axis=1) > 0).all(axis=1)
            say(f"  tokens whose four near logits are all distinct: {int(distinct.sum())} of {T}")
    _layers.pop((1, None), None)
    ctx.synth_layer(1, SEED, None)  # restore the synthetic router for later tests


def survivor_count(lg):
    """Experts at or above the smallest of the eight group maxima (a group is
    the 32 experts l + 64 j of lanes l = 8 g .. 8 g + 7), per token: the
    candidates the GPU top-8 sorts."""
    v = lg[:, :256]
    g = v.reshape(-1, 4, 8, 8).max(axis=(1, 3)).min(axis=1)
    return (v >= g[:, None]).sum(axis=1)


def survivor_bias(S, seed):
    """A router bias (steps of 25, far above the dot's few units) that orders
    the experts so that exactly S survive: group 0's largest expert is the
    S-th largest, and every other group has one among the S - 1 above it."""
    rng = np.random.default_rng(seed)
    e = np.arange(256)
    grp = (e & 63) >> 3
    firsts = [int(rng.choice(e[grp == g])) for g in range(1, 8)]
    others = [int(i) for i in rng.permutation(e[grp != 0]) if i not in firsts]
    g0 = [int(i) for i in rng.permutation(e[grp == 0])]
    top = firsts + others[:S - 8]
    rng.shuffle(top)
    order = top + g0[:1] + others[S - 8:] + g0[1:]
    bias = np.empty(256, np.float32)
    bias[order] = 25.0 * (255 - np.arange(256, dtype=np.float32))
    return bias, order


@pytest.mark.parametrize("S,tie", [(33, False), (33, True), (64, False), (64, True), (65, False), (100, False)])
@pytest.mark.parametrize("T", [1, 5, 64])
def test_topk_survivor_counts(ctx, torch_cuda, S, tie, T):
    # 33..64 survivors take the 64-wide register sort (T = 1 decode, T > 1
    # decode, and the prefill top-8), more take the fallbacks (ranks counted in
    # LDS at T = 1, rounds of wave maxima otherwise).  "tie": the experts ranked
    # 3rd and 4th get one router row and one bias, so their logits are equal and
    # T = 1 takes its 64-bit sort
    say(f"top-8 with {S} survivors{' and a tie' if tie else ''}, T={T}")
    bias, order = survivor_bias(S, 900 + S)
    L = O.SynthLayer(SEED, 1, bias=bias)
    if tie:
        a, b = order[2], order[3]
        bias[b] = bias[a]
        L.bias = bias
        R = L.router.copy()
        R[b] = R[a]
        L.router = np.ascontiguousarray(R, np.float32)
    x = O.gen_x(SEED, 700 + T, T)
    lg = O.router(x, L.router, L.bias)
    assert (survivor_count(lg) == S).all()
    if tie:
        assert (lg[:, order[2]] == lg[:, order[3]]).all()
    ctx.synth_layer(1, SEED, bias)
    if tie:
        ctx.set_dense(1, router=L.router)
    xd = torch_cuda.from_numpy(x).cuda()
    y = torch_cuda.empty_like(xd)
    ctx.forward_normed(1, xd, y, T)
    torch_cuda.cuda.synchronize()
    g = ctx.routing(T)
    g["logits"] = ctx.logits(T)
    g["out"] = y.cpu().numpy()
    check_layer(L, g, x)
    ctx.synth_layer(1, SEED, None)  # restore the synthetic router for later tests


class PackLayer:
    """Oracle view of a layer loaded from a pack (same bytes the loader uploads)."""

    def __init__(self, t):
        self.router = np.ascontiguousarray(np.vstack([t["router"], t["sh_gate"][None]]), np.float32)
        self.sh_gu = np.ascontiguousarray(np.concatenate([t["sh_gate_proj"].reshape(-1), t["sh_up"].reshape(-1)]))
        self.sh_dn = np.ascontiguousarray(t["sh_down"].reshape(-1))
        self.bias = None
        self._ex = t["experts"]

    def experts(self, ids):
        return {int(e): np.ascontiguousarray(self._ex[int(e)]) for e in np.unique(ids)}


def test_pack_loader(ctx, torch_cuda, tmp_path):
    import packfile as PF
    say("weight pack: blk.3 of a synthetic pack -> context layer 1, norm + residual")
    t = PF.synth_moe_tensors(1234)
    path = tmp_path / "moe.pack"
    PF.write_pack(path, PF.pack_entries(3, t))
    ctx.load_pack(path, 3, 1, 1)
    L = PackLayer(t)
    for T in (1, 20):
        x = O.gen_x(SEED, 500 + T, T)
        xd = torch_cuda.from_numpy(x).cuda()
        y = torch_cuda.empty_like(xd)
        ctx.forward(1, xd, y, T)
        torch_cuda.cuda.synchronize()
        g = ctx.routing(T)
        o = O.moe_layer(L, x, norm=True, residual=True, post_norm=t["post_norm"])
        assert np.array_equal(ctx.logits(T).view(np.uint32), o["logits"].view(np.uint32)), "router logits differ"
        assert np.array_equal(g["ids"], o["ids"])
        e_out, e_sd = rel_l2(y.cpu().numpy(), o["out"]), rel_l2(g["sd"], o["sd"])
        say(f"  T={T} out rel-L2 {e_out:.2e}  shared rel-L2 {e_sd:.2e}")
        assert e_out <= TOL and e_sd <= TOL
    # errors come back as codes with a message, nothing is half-loaded into a ready layer
    bad = tmp_path / "bad.pack"
    PF.write_pack(bad, PF.pack_entries(3, t), magic=b"NOTAPACK")
    with pytest.raises(qe_moe.QeError, match="bad magic"):
        ctx.load_pack(bad, 3, 1, 1)
    with pytest.raises(qe_moe.QeError, match="missing blk.4.post_norm"):
        ctx.load_pack(path, 4, 1, 1)
    PF.write_pack(bad, PF.pack_entries(3, t, {"sh_up": PF.F_Q6}))
    with pytest.raises(qe_moe.QeError, match="sh_up has format 2"):
        ctx.load_pack(bad, 3, 1, 1)
    with pytest.raises(qe_moe.QeError, match="cannot open"):
        ctx.load_pack(tmp_path / "none.pack", 3, 1, 1)
    _layers.pop((1, None), None)
    ctx.synth_layer(1, SEED, None)


def test_dispatch_on_reference_routing_records(ctx, torch_cuda):
    import os
    torch = torch_cuda
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "routing_records.npz"))
    for name in sorted({k.rsplit("_", 1)[0] for k in fx.files}):
        say(f"dispatch fixture {name}")
        ids = torch.from_numpy(fx[name + "_ids"].astype(np.int32)).cuda()
        T = ids.shape[0]
        ctx.dispatch(ids, T)
        r = ctx.routing(T)
        assert np.array_equal(r["off"], fx[name + "_off"]) and np.array_equal(r["pairs"], fx[name + "_pairs"])


def test_dispatch_extremes(ctx, torch_cuda):
    torch = torch_cuda
    rng = np.random.default_rng(9)
    # all tokens on the same 8 experts (maximal skew), and the maximum T
    for T, ids in ((8192, np.tile(np.arange(8, dtype=np.int32)[::-1], (8192, 1))),
                   (8192, np.stack([rng.choice(256, 8, replace=False) for _ in range(8192)]).astype(np.int32)),
                   (3, np.array([[255, 0, 1, 2, 3, 4, 5, 6]] * 3, np.int32))):
        say(f"dispatch extreme T={T}")
        ctx.dispatch(torch.from_numpy(ids).cuda(), T)
        r = ctx.routing(T)
        off, pairs = O.dispatch(ids)
        assert np.array_equal(r["off"], off) and np.array_equal(r["pairs"], pairs)


@pytest.mark.parametrize("T", [1, 8])
def test_cfg2_stack_40_layers(torch_cuda, T):
    """Config 2 at its size: 40 layers, all 40 x 256 experts resident (18.1 GB of
    arena, so layers 10..39 sit above 4 GB), x_{l+1} = x_l + MoE_l(RMSNorm(x_l)).

    * forward_stack(0, 40) in one persistent launch equals the same chain run
      layer by layer through qe_moe_forward, bit for bit (same kernel, same
      per-layer arithmetic, the 40-layer tag/ping-pong sequence in between);
    * every layer of that chain is checked against the oracle on the same input
      (teacher forcing: the oracle consumes the GPU's x_l), logits and ids bit
      for bit, the output and the shared term within 1e-3;
    * the end-to-end drift against the pure oracle chain is reported, and bounded
      by 1e-3 when no layer's routing differs between the two chains.
    """
    torch = torch_cuda
    n, seed = 40, SEED + 4040
    m = qe_moe.MoE(n_layers=n, t_max=8)
    try:
        say(f"config 2: 40 layers, T={T}: synthesising the arena")
        for l in range(n):
            m.synth_layer(l, seed, None)
        x0 = O.gen_x(seed, 900 + T, T)
        x_in = torch.from_numpy(x0).cuda()
        x_out = torch.empty_like(x_in)
        m.forward_stack(0, n, x_in, x_out, T)
        torch.cuda.synchronize()
        m.check()
        stack_gpu = x_out.cpu().numpy()
        h, h_orc, flips = x0, x0, 0
        for l in range(n):
            L = O.SynthLayer(seed, l)
            xi = torch.from_numpy(h).cuda()
            yo = torch.empty_like(xi)
            m.forward(l, xi, yo, T)
            torch.cuda.synchronize()
            g = m.routing(T)
            g["logits"] = m.logits(T)
            g["out"] = yo.cpu().numpy()
            say(f"  layer {l}")
            check_layer(L, g, h, norm=True)
            o_chain = O.moe_layer(L, h_orc, norm=True, residual=True)
            flips += int(not np.array_equal(o_chain["ids"], g["ids"]))
            h, h_orc = g["out"], o_chain["out"]
            del L
        assert np.array_equal(stack_gpu.view(np.uint32), h.view(np.uint32)), "stack differs from the per-layer chain"
        drift = rel_l2(stack_gpu, h_orc)
        say(f"  end-to-end drift vs the oracle chain: rel-L2 {drift:.2e}, layers with other routing: {flips}")
        if flips == 0:
            assert drift <= TOL
    finally:
        m.close()


@pytest.mark.parametrize("T", [2, 3, 4, 5, 6, 7])
def test_short_stack_every_batch(torch_cuda, T):
    """A 3-layer persistent launch at each batch size the T <= 8 kernel takes
    between the two the 40-layer test covers: x crosses the exchange 2, 4, 6, 8,
    10, 12 or 14 words per thread (polled in rounds of 8, then 4 and 2), and the
    stack equals the layer-by-layer chain bit for bit, each layer matching the
    oracle on the GPU's own input.  A second launch on the same input repeats
    the first bit for bit (the routed down sums per lane group in LDS, the
    exchanges: nothing depends on timing)."""
    torch = torch_cuda
    n, seed = 3, SEED + 3300 + T
    m = qe_moe.MoE(n_layers=n, t_max=8)
    try:
        for l in range(n):
            m.synth_layer(l, seed, None)
        x0 = O.gen_x(seed, 910 + T, T)
        x_in = torch.from_numpy(x0).cuda()
        x_out = torch.empty_like(x_in)
        say(f"{n}-layer stack, T={T}")
        m.forward_stack(0, n, x_in, x_out, T)
        torch.cuda.synchronize()
        m.check()
        stack_gpu = x_out.cpu().numpy()
        m.forward_stack(0, n, x_in, x_out, T)
        torch.cuda.synchronize()
        m.check()
        assert np.array_equal(x_out.cpu().numpy().view(np.uint32), stack_gpu.view(np.uint32)), "repeat launch differs"
        h = x0
        for l in range(n):
            L = O.SynthLayer(seed, l)
            xi = torch.from_numpy(h).cuda()
            yo = torch.empty_like(xi)
            m.forward(l, xi, yo, T)
            torch.cuda.synchronize()
            g = m.routing(T)
            g["logits"] = m.logits(T)
            g["out"] = yo.cpu().numpy()
            check_layer(L, g, h, norm=True)
            h = g["out"]
            del L
        assert np.array_equal(stack_gpu.view(np.uint32), h.view(np.uint32)), "stack differs from the per-layer chain"
    finally:
        m.close()


def test_errors_are_reported(ctx, torch_cuda):
    torch = torch_cuda
    x = torch.zeros(1, 2048, device="cuda")
    with pytest.raises(qe_moe.QeError) as e:
        ctx.forward_normed(0, x, x, 1)
    assert e.value.code == qe_moe.QE_ERR_ARG
    with pytest.raises(qe_moe.QeError):
        ctx.forward_normed(0, x, torch.empty_like(x), 8193)
    with pytest.raises(qe_moe.QeError):
        ctx.forward_normed(5, x, torch.empty_like(x), 1)
