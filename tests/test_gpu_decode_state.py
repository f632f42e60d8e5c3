"""GPU tests of the decode path's state across launches (needs an MI355X).

* The exchanged words carry the launch counter modulo 65536 in their tags; a
  word that no launch rewrote for a multiple of 65536 launches must not pass a
  poll.  The regression runs launches across the counter's wrap with batch
  sizes that write different exchange slots, and checks every one against the
  oracle.
* A poll that gives up is reported to the caller (QE_ERR_STATE), once.
* A forward call on a layer whose tensors were not all set is refused.
"""
import numpy as np
import pytest

import oracle as O
import qe_moe

pytestmark = pytest.mark.gpu
SEED = 0xE90C
TOL = 1e-3


def say(msg):
    print(msg, flush=True)


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b.astype(np.float64)), 1e-30))


def run_and_check(torch, m, L, x):
    T = x.shape[0]
    xd = torch.from_numpy(x).cuda()
    y = torch.empty_like(xd)
    m.forward_normed(0, xd, y, T)
    torch.cuda.synchronize()
    g = m.routing(T)
    o = O.moe_layer(L, x)
    assert np.array_equal(m.logits(T).view(np.uint32), o["logits"].view(np.uint32)), "router logits differ"
    assert np.array_equal(g["ids"], o["ids"]), "routing ids differ"
    assert np.array_equal(g["pairs"], o["pairs"]) and np.array_equal(g["off"], o["off"]), "dispatch differs"
    e = rel_l2(y.cpu().numpy(), o["out"])
    assert e <= TOL, e
    return e


def test_decode_epoch_wrap(torch_cuda):
    torch = torch_cuda
    m = qe_moe.MoE(n_layers=1, t_max=8)
    try:
        L = O.SynthLayer(SEED, 0, bias=O.gen_zipf_bias(SEED, 0, 1.0))
        m.synth_layer(0, SEED, L.bias)
        # epoch 0: a T = 8 launch writes the int8-h words of 64 pairs with tags of epoch 0
        say("epoch wrap: T=8 at epoch 0")
        run_and_check(torch, m, L, O.gen_x(SEED, 1, 8))
        # jump to the last epoch before the wrap; the launch there crosses it, and the
        # next T = 8 launch polls tags equal to those stale epoch-0 words
        m.debug_set_epoch(65535)
        seq = [1, 8, 1, 8, 5, 1, 8]
        for i, T in enumerate(seq):
            say(f"epoch wrap: launch {i} at epoch {65535 + i}, T={T}")
            run_and_check(torch, m, L, O.gen_x(SEED, 10 + i, T))
        m.check()
    finally:
        m.close()


def test_decode_poll_timeout_is_reported(torch_cuda):
    # A poll cap of one read makes exchange waits give up; the kernel still runs
    # to its end, and the next call reports it.  The forcing launch is a two-layer
    # stack at T = 8: the second layer's x is polled by each workgroup as soon as
    # it has published its own rows of the first layer's, microseconds before the
    # slowest workgroup publishes its rows, so a first read misses.  (A single
    # layer at T = 1 can find every word in place at the first read.)
    torch = torch_cuda
    m = qe_moe.MoE(n_layers=2, t_max=8)
    try:
        L = O.SynthLayer(SEED, 0)
        for l in range(2):
            m.synth_layer(l, SEED, None)
        x = O.gen_x(SEED, 3, 1)
        xd = torch.from_numpy(x).cuda()
        y = torch.empty_like(xd)
        x8 = torch.from_numpy(O.gen_x(SEED, 4, 8)).cuda()
        y8 = torch.empty_like(x8)
        m.debug_set_spin_cap(1)
        say("poll timeout: forced by a one-read cap, 2-layer stack at T=8")
        err = None
        for _ in range(5):
            m.forward_stack(0, 2, x8, y8, 8)  # launches; its own timeout is not known yet
            try:
                m.check()
            except qe_moe.QeError as ex:
                err = ex
                break
        assert err is not None and err.code == qe_moe.QE_ERR_STATE and "timed out" in str(err)
        m.check()  # reported once, then cleared
        for _ in range(5):
            try:  # the next forward call reports it, before launching
                m.forward_stack(0, 2, x8, y8, 8)
                torch.cuda.synchronize()
                m.forward_normed(0, xd, y, 1)
            except qe_moe.QeError as ex:
                assert ex.code == qe_moe.QE_ERR_STATE and "timed out" in str(ex)
                break
        else:
            pytest.fail("no forward call reported the forced timeout")
        m.debug_set_spin_cap(0)  # back to the default cap
        torch.cuda.synchronize()
        m.check()
        say("poll timeout: default cap again, output checked")
        run_and_check(torch, m, L, x)
    finally:
        m.close()


def test_fused_prefill_wait_timeout_is_reported(torch_cuda):
    # From 32 to 4095 tokens the routed gate/up, routed down and shared down run as
    # one launch whose down workgroups wait for their item's gate/up workgroups.
    # The grid order usually finds those done at the first read, so the test hook
    # makes every wait expect one workgroup more than exists, and a cap of one read
    # lets each give up at once (the kernel still runs to its end); the next call
    # reports it, once, with the prefill call's number.  Then the hook and the cap
    # back to their defaults, and the output checked against the oracle.
    torch = torch_cuda
    T = 512
    m = qe_moe.MoE(n_layers=1, t_max=T)
    try:
        L = O.SynthLayer(SEED, 0)
        m.synth_layer(0, SEED, None)
        x = O.gen_x(SEED, 7, T)
        xd = torch.from_numpy(x).cuda()
        y = torch.empty_like(xd)
        m.debug_set_spin_cap(1)
        m.debug_fused_wait_extra(1)
        say("fused prefill wait: forced by the wait hook and a one-read cap, T=512")
        err = None
        for _ in range(5):
            m.forward_normed(0, xd, y, T)
            try:
                m.check()
            except qe_moe.QeError as ex:
                err = ex
                break
        assert err is not None and err.code == qe_moe.QE_ERR_STATE and "prefill call" in str(err)
        m.check()  # reported once, then cleared
        m.debug_fused_wait_extra(0)
        m.debug_set_spin_cap(0)
        m.forward_normed(0, xd, y, T)
        m.check()
        o = O.moe_layer(L, x)
        g = m.routing(T)
        assert np.array_equal(g["ids"], o["ids"])
        e = float(np.linalg.norm(y.cpu().numpy().astype(np.float64) - o["out"]) / np.linalg.norm(o["out"]))
        say(f"  default cap again: out rel-L2 {e:.2e}")
        assert e <= 1e-3
    finally:
        m.close()


def test_layer_readiness(torch_cuda):
    torch = torch_cuda
    m = qe_moe.MoE(n_layers=1, t_max=8)
    try:
        x = torch.zeros(1, 2048, device="cuda")
        y = torch.empty_like(x)
        say("readiness: nothing set")
        with pytest.raises(qe_moe.QeError, match="post_norm, router, sh_gu, sh_down, 256 experts") as e:
            m.forward(0, x, y, 1)
        assert e.value.code == qe_moe.QE_ERR_STATE
        L = O.SynthLayer(SEED, 0)
        m.set_dense(0, post_norm=np.ones(2048, np.float32))
        with pytest.raises(qe_moe.QeError, match="router, sh_gu, sh_down, 256 experts"):
            m.forward(0, x, y, 1)
        m.set_dense(0, router=L.router, sh_gu=L.sh_gu, sh_down=L.sh_dn)
        with pytest.raises(qe_moe.QeError, match="lacks 256 experts"):
            m.forward(0, x, y, 1)
        blobs = torch.zeros(128 * qe_moe.EXPERT_BYTES, dtype=torch.uint8, device="cuda")
        m.upload_experts(0, 0, blobs, on_device=True)
        with pytest.raises(qe_moe.QeError, match="lacks 128 experts"):
            m.forward(0, x, y, 1)
        m.upload_experts(0, 128, blobs, on_device=True)
        m.forward(0, x, y, 1)
        m.check()
    finally:
        m.close()
