"""GPU parity of the IQ4_NL converter against the CPU oracle (needs an MI355X).

The oracle restates ggml's IQ4_NL quantizer as the reference converter calls
it (engine/qconv.cpp:91-98, :202-227); the GPU kernel must reproduce its
bytes exactly: same fp16 scales, same code nibbles, for every source type.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
import qe_moe

pytestmark = pytest.mark.gpu
KV = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)


def say(msg):
    print(msg, flush=True)


def d2h(ptr, nbytes):
    buf = np.empty(nbytes, np.uint8)
    hip = ctypes.CDLL("libamdhip64.so")
    assert hip.hipMemcpy(ctypes.c_void_p(buf.ctypes.data), ctypes.c_void_p(ptr), ctypes.c_size_t(nbytes), 2) == 0
    return buf


def special_rows(rng, rows, cols):
    """Random blocks over 12 decades, with the edge cases of the quantizer planted."""
    nb = rows * cols // 32
    x = (rng.standard_normal((nb, 32)) * 10.0 ** rng.uniform(-6, 3, (nb, 1))).astype(np.float32)
    k = 0

    def plant(v):
        nonlocal k
        x[k] = v
        k += 1

    plant(np.zeros(32))                                  # zero block: scale 0, codes 8
    for s in (2.0 ** -9, -0.5, 3.0):                     # exact fits of the codebook
        plant(KV[rng.integers(0, 16, 32)] * s)
        x[k - 1, 3] = -127 * s
    for _ in range(4):                                   # +A and -A both present
        v = rng.standard_normal(32)
        j = int(np.argmax(np.abs(v)))
        v[(j + 7) % 32] = -v[j]
        plant(v)
    for a in (9e-16, 1e-15, 1.1e-15, 1e-39, 1e-30, 6e-8):  # around the 1e-15 threshold; fp16 scale underflow
        v = np.zeros(32)
        v[int(rng.integers(0, 32))] = a
        v[int(rng.integers(0, 32))] = -a / 3
        plant(v)
    mids = (KV[:-1] + KV[1:]) / 2                        # values on bracket midpoints
    plant(np.resize(mids, 32) / 127.0)
    plant(np.full(32, 0.25))                             # constant block
    plant(np.linspace(-1, 1, 32))
    return x.reshape(rows, cols)


def as_source(x, src_type, rng):
    rows, cols = x.shape
    nb = rows * cols // 32
    if src_type == O.SRC_F32:
        return x
    if src_type == O.SRC_F16:
        return x.astype(np.float16)
    if src_type == O.SRC_BF16:
        return (x.view(np.uint32) >> 16).astype(np.uint16)
    xb = x.reshape(nb, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / 127).astype(np.float16)
    di = np.where(d.astype(np.float32) > 0, 1 / np.maximum(d.astype(np.float32), 1e-30), 0)
    q = np.clip(np.rint(xb * di[:, None]), -127, 127).astype(np.int8)
    return np.concatenate([d.view(np.uint8).reshape(nb, 2), q.view(np.uint8)], axis=1)


@pytest.mark.parametrize("src_type", [O.SRC_F32, O.SRC_F16, O.SRC_BF16, O.SRC_Q8_0])
@pytest.mark.parametrize("rows,cols", [(512, 2048), (2048, 512), (3, 256)])
def test_nl4_rows_bit_exact(torch_cuda, src_type, rows, cols):
    torch = torch_cuda
    say(f"nl4 rows: type {src_type}, {rows} x {cols}")
    rng = np.random.default_rng(rows * 7 + cols + src_type)
    src = np.ascontiguousarray(as_source(special_rows(rng, rows, cols), src_type, rng))
    want = O.nl4_quantize_rows(src, src_type, rows, cols)
    s_dev = torch.from_numpy(src.view(np.uint8).reshape(-1).copy()).cuda()
    out = torch.full((rows * O.nl4_row_bytes(cols),), 0xEE, dtype=torch.uint8, device="cuda")
    qe_moe.nl4_quantize_rows(s_dev, src_type, rows, cols, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(rows, -1)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} bytes differ, first at row/byte {bad[:4].tolist()}"


def test_nl4_rows_errors(torch_cuda):
    torch = torch_cuda
    a = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    with pytest.raises(qe_moe.QeError, match="bad argument"):
        qe_moe.nl4_quantize_rows(a, O.SRC_F32, 1, 100, a)
    with pytest.raises(qe_moe.QeError, match="unsupported source type 2"):
        qe_moe.nl4_quantize_rows(a, 2, 1, 256, a)
    qe_moe.nl4_quantize_rows(a, O.SRC_F32, 0, 256, a)  # no rows: nothing to do


def test_convert_experts_layer_q8_0(torch_cuda):
    """blk.N.ffn_{gate,up,down}_exps in Q8_0 (the reference converter's input) -> the arena blob of a layer."""
    torch = torch_cuda
    say("convert_experts: one layer of Q8_0 experts")
    g = torch.Generator(device="cuda")
    g.manual_seed(20261201)

    def q8(nblk):
        t = torch.randint(0, 256, (nblk, 34), dtype=torch.uint8, device="cuda", generator=g)
        d = (torch.rand(nblk, device="cuda", generator=g) * 0.02).half()
        t[:, :2] = d.view(torch.uint8).view(nblk, 2)
        return t

    gate, up = q8(256 * 512 * 64), q8(256 * 512 * 64)
    down = q8(256 * 2048 * 16)
    m = qe_moe.MoE(n_layers=2, t_max=16)
    try:
        m.synth_layer(1, 0xC0FFEE, None)  # dense weights from the generator; experts replaced below
        m.convert_experts(1, gate, up, down, qe_moe.SRC_Q8_0)
        torch.cuda.synchronize()
        hg, hu, hd = (t.cpu().numpy() for t in (gate, up, down))
        arena = d2h(m.arena_ptr(1), 256 * O.EXPERT_BYTES).reshape(256, O.EXPERT_BYTES)
        rng = np.random.default_rng(3)
        for e in sorted({0, 1, 2, 127, 128, 254, 255, *rng.integers(3, 254, 9).tolist()}):
            want = O.convert_expert(hg, hu, hd, O.SRC_Q8_0, e)
            assert np.array_equal(arena[e], want), f"expert {e} differs"
        say("  16 experts bit-exact; forward over the converted layer")
        # the converted layer runs through the forward path like any arena layer
        L = O.SynthLayer(0xC0FFEE, 1)
        L.experts = lambda ids: {int(e): np.ascontiguousarray(arena[int(e)]) for e in np.unique(ids)}
        x = O.gen_x(0xC0FFEE, 77, 3)
        xd = torch.from_numpy(x).cuda()
        y = torch.empty_like(xd)
        m.forward(1, xd, y, 3)
        torch.cuda.synchronize()
        o = O.moe_layer(L, x, norm=True, residual=True)
        r = m.routing(3)
        assert np.array_equal(r["ids"], o["ids"])
        e_out = float(np.linalg.norm(y.cpu().numpy().astype(np.float64) - o["out"]) / np.linalg.norm(o["out"]))
        say(f"  out rel-L2 {e_out:.2e}")
        assert e_out <= 1e-3
    finally:
        m.close()
