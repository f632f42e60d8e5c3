"""numpy wrappers over liboracle (oracle/qe_oracle.cpp) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, always as the checker (or the timed CPU baseline), never as the
product path.  See qe_oracle.cpp for the reference file:line each function
restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqe_oracle.so")

D, NE, K, FF = 2048, 256, 8, 512
ROUTER_ROWS = 257
EXPERT_BYTES = 1769472
SH_GU_BYTES = 1024 * 2176
SH_DN_BYTES = 2048 * 544

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, u64, u32, f32, f64 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64,
                                        ctypes.c_uint32, ctypes.c_float, ctypes.c_double)
    sig = {
        "orc_gen_expert": (None, [u64, i32, i32, vp]),
        "orc_gen_router": (None, [u64, i32, vp]),
        "orc_gen_q8": (None, [u64, i32, i32, vp]),
        "orc_gen_x": (None, [u64, i32, vp, i64]),
        "orc_gen_zipf_bias": (None, [u64, i32, f64, vp]),
        "orc_f32_to_f16": (ctypes.c_uint16, [f32]),
        "orc_f16_to_f32": (f32, [ctypes.c_uint16]),
        "orc_normal": (f64, [u64, u64]),
        "orc_log_unit": (f64, [f64]),
        "orc_cos_turns": (f64, [f64]),
        "orc_stream_key": (u64, [u64, u32, u32, u32]),
        "orc_draw": (u64, [u64, u64]),
        "orc_quant_x": (None, [vp, i32, vp, vp]),
        "orc_quant_x_avx2": (None, [vp, i32, vp, vp]),
        "orc_dot_nl4": (f32, [vp, i32, vp, vp]),
        "orc_dot_nl4_avx2": (f32, [vp, i32, vp, vp]),
        "orc_dot_nl4_x4_avx2": (None, [vp, i32, vp, vp, i32, vp]),
        "orc_canon_dot": (f32, [vp, vp]),
        "orc_canon_sumsq": (f32, [vp]),
        "orc_rmsnorm": (None, [vp, vp, i32, vp]),
        "orc_router": (None, [vp, vp, vp, i32, vp]),
        "orc_topk": (None, [vp, i32, vp, vp, vp]),
        "orc_dispatch": (None, [vp, i32, vp, vp]),
        "orc_shared": (None, [vp, i32, vp, vp, vp, vp]),
        "orc_routed": (None, [vp, i32, vp, vp, vp, vp, vp, i32]),
        "orc_combine": (None, [vp, vp, vp, vp, i32, vp]),
        "orc_baseline_layer": (f64, [vp, vp, vp, vp, vp, vp, vp, i32, i32, vp]),
        "orc_nl4_nearest": (i32, [f32]),
        "orc_nl4_block": (f32, [vp, vp, vp]),
        "orc_nl4_quantize_rows": (i32, [vp, i32, i64, i32, vp]),
        "orc_convert_expert": (i32, [vp, vp, vp, i32, i32, vp]),
        "orc_set_threads": (None, [i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    _lib = lib
    return lib


def _p(a):
    if a is None:
        return None
    assert isinstance(a, np.ndarray) and a.flags["C_CONTIGUOUS"], type(a)
    return a.ctypes.data


# ---------------- generators ----------------
def gen_expert(seed, layer, expert):
    out = np.empty(EXPERT_BYTES, np.uint8)
    load().orc_gen_expert(seed, layer, expert, _p(out))
    return out


def gen_router(seed, layer):
    out = np.empty((ROUTER_ROWS, D), np.float32)
    load().orc_gen_router(seed, layer, _p(out))
    return out


def gen_sh_gu(seed, layer):
    out = np.empty(SH_GU_BYTES, np.uint8)
    load().orc_gen_q8(seed, layer, 0, _p(out))
    return out


def gen_sh_dn(seed, layer):
    out = np.empty(SH_DN_BYTES, np.uint8)
    load().orc_gen_q8(seed, layer, 1, _p(out))
    return out


def gen_x(seed, inst, T):
    out = np.empty((T, D), np.float32)
    load().orc_gen_x(seed, inst, _p(out), T * D)
    return out


def gen_zipf_bias(seed, layer, s):
    out = np.empty(NE, np.float32)
    load().orc_gen_zipf_bias(seed, layer, s, _p(out))
    return out


# ---------------- primitives ----------------
def quant_x(x, avx2=False):
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.int8)
    s = np.empty(x.size // 32, np.float32)
    (load().orc_quant_x_avx2 if avx2 else load().orc_quant_x)(_p(x), x.size, _p(q), _p(s))
    return q, s


def dot_nl4(row, cols, xq, xs, avx2=False):
    f = load().orc_dot_nl4_avx2 if avx2 else load().orc_dot_nl4
    return f(_p(np.ascontiguousarray(row)), cols, _p(np.ascontiguousarray(xq)), _p(np.ascontiguousarray(xs)))


def dot_nl4_x4(row, cols, xqs, xss):
    """row . x_t for up to four quantised activation rows, weights decoded once per block."""
    n = len(xqs)
    xqs = [np.ascontiguousarray(q) for q in xqs]
    xss = [np.ascontiguousarray(s) for s in xss]
    qp = (ctypes.c_void_p * 4)(*[q.ctypes.data for q in xqs], *([None] * (4 - n)))
    sp = (ctypes.c_void_p * 4)(*[s.ctypes.data for s in xss], *([None] * (4 - n)))
    out = np.zeros(4, np.float32)
    load().orc_dot_nl4_x4_avx2(_p(np.ascontiguousarray(row)), cols, ctypes.cast(qp, ctypes.c_void_p),
                               ctypes.cast(sp, ctypes.c_void_p), n, _p(out))
    return out[:n]


def canon_dot(a, b):
    return load().orc_canon_dot(_p(np.ascontiguousarray(a, np.float32)), _p(np.ascontiguousarray(b, np.float32)))


def canon_sumsq(x):
    return load().orc_canon_sumsq(_p(np.ascontiguousarray(x, np.float32)))


def rmsnorm(x, w=None):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    load().orc_rmsnorm(_p(x), _p(w), x.shape[0], _p(out))
    return out


def router(xn, W, bias=None):
    T = xn.shape[0]
    out = np.empty((T, ROUTER_ROWS), np.float32)
    load().orc_router(_p(np.ascontiguousarray(xn, np.float32)), _p(W), _p(bias), T, _p(out))
    return out


def topk(logits):
    T = logits.shape[0]
    ids = np.empty((T, K), np.int32)
    wts = np.empty((T, K), np.float32)
    shg = np.empty(T, np.float32)
    load().orc_topk(_p(np.ascontiguousarray(logits, np.float32)), T, _p(ids), _p(wts), _p(shg))
    return ids, wts, shg


def dispatch(ids):
    ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
    T = ids.size // K
    off = np.empty(NE + 1, np.int32)
    pairs = np.empty(T * K, np.int32)
    load().orc_dispatch(_p(ids), T, _p(off), _p(pairs))
    return off, pairs


def shared(xn, sh_gu, sh_dn, want_h=False):
    T = xn.shape[0]
    sd = np.empty((T, D), np.float32)
    h = np.empty((T, 512), np.float32) if want_h else None
    load().orc_shared(_p(np.ascontiguousarray(xn, np.float32)), T, _p(sh_gu), _p(sh_dn), _p(sd), _p(h))
    return (sd, h) if want_h else sd


def routed(xn, ids, wts, experts: dict, want_h=False, avx2=True):
    """experts: {expert_id: uint8 blob}; every routed id must be present."""
    T = xn.shape[0]
    ptrs = (ctypes.c_void_p * NE)()
    for e, blob in experts.items():
        ptrs[e] = blob.ctypes.data
    for e in np.unique(ids):
        assert int(e) in experts, f"expert {e} missing"
    yp = np.empty((T * K, D), np.float32)
    h = np.empty((T * K, FF), np.float32) if want_h else None
    load().orc_routed(_p(np.ascontiguousarray(xn, np.float32)), T, _p(np.ascontiguousarray(ids, np.int32)),
                      _p(np.ascontiguousarray(wts, np.float32)), ctypes.cast(ptrs, ctypes.c_void_p), _p(yp), _p(h),
                      int(avx2))
    return (yp, h) if want_h else yp


def combine(x2, shg, sd, yp):
    T = sd.shape[0]
    out = np.empty((T, D), np.float32)
    load().orc_combine(_p(x2), _p(shg), _p(sd), _p(yp), T, _p(out))
    return out


class SynthLayer:
    """Host copy of one synthetic layer's dense weights; experts generated on demand."""

    def __init__(self, seed, layer, bias=None):
        self.seed, self.layer = seed, layer
        self.router = gen_router(seed, layer)
        self.sh_gu = gen_sh_gu(seed, layer)
        self.sh_dn = gen_sh_dn(seed, layer)
        self.bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self._experts = {}

    def experts(self, ids):
        for e in np.unique(ids):
            e = int(e)
            if e not in self._experts:
                self._experts[e] = gen_expert(self.seed, self.layer, e)
        return {int(e): self._experts[int(e)] for e in np.unique(ids)}


def moe_layer(L: SynthLayer, x, norm=False, residual=False, post_norm=None):
    """The whole block on T tokens: returns dict with every intermediate."""
    x = np.ascontiguousarray(x, np.float32)
    xn = rmsnorm(x, post_norm if post_norm is not None else np.ones(D, np.float32)) if norm else x
    logits = router(xn, L.router, L.bias)
    ids, wts, shg = topk(logits)
    off, pairs = dispatch(ids)
    sd = shared(xn, L.sh_gu, L.sh_dn)
    yp = routed(xn, ids, wts, L.experts(ids))
    out = combine(x if residual else None, shg, sd, yp)
    return dict(xn=xn, logits=logits, ids=ids, wts=wts, shg=shg, off=off, pairs=pairs, sd=sd, yp=yp, out=out)


def baseline_layer(x2, post_norm, L: SynthLayer, experts_ptrs, T, threads):
    out = np.empty((T, D), np.float32)
    sec = load().orc_baseline_layer(_p(x2), _p(post_norm), _p(L.router), _p(L.bias), _p(L.sh_gu), _p(L.sh_dn),
                                    ctypes.cast(experts_ptrs, ctypes.c_void_p), T, threads, _p(out))
    return sec, out


# ---------------------------------------------------------------------------
# IQ4_NL converter (qe_oracle.cpp: ggml's quantizer as the reference converter
# calls it, engine/qconv.cpp:17-43, :91-98, :202-227)
# ---------------------------------------------------------------------------
SRC_F32, SRC_F16, SRC_Q8_0, SRC_BF16 = 0, 1, 8, 30
SRC_BLOCK_BYTES = {SRC_F32: 128, SRC_F16: 64, SRC_Q8_0: 34, SRC_BF16: 64}


def nl4_row_bytes(cols):
    return cols // 2 + cols // 32 * 2


def nl4_nearest(a):
    return load().orc_nl4_nearest(float(a))


def nl4_block(x):
    """One 32-element block -> (fp16 scale bits, 16 code bytes, fp32 scale)."""
    x = np.ascontiguousarray(x, np.float32)
    assert x.shape == (32,)
    d16 = np.zeros(1, np.uint16)
    codes = np.zeros(16, np.uint8)
    d = load().orc_nl4_block(_p(x), _p(d16), _p(codes))
    return int(d16[0]), codes, float(d)


def nl4_quantize_rows(src, src_type, rows, cols):
    """src: the ggml tensor's bytes (any dtype view, contiguous blocks)."""
    src = np.ascontiguousarray(src)
    assert src.nbytes == rows * cols // 32 * SRC_BLOCK_BYTES[src_type]
    out = np.empty((rows, nl4_row_bytes(cols)), np.uint8)
    assert load().orc_nl4_quantize_rows(_p(src), src_type, rows, cols, _p(out)) == 0
    return out


def convert_expert(gate, up, down, src_type, e):
    out = np.empty(EXPERT_BYTES, np.uint8)
    gate, up, down = (np.ascontiguousarray(a) for a in (gate, up, down))
    assert load().orc_convert_expert(_p(gate), _p(up), _p(down), src_type, e, _p(out)) == 0
    return out


def nl4_dequant_rows(rows_u8, cols):
    """NL4 rows -> fp32 (codebook value * fp16 scale), for error statistics."""
    nb = cols // 32
    r = np.ascontiguousarray(rows_u8).reshape(-1, nl4_row_bytes(cols))
    codes = r[:, : cols // 2].reshape(-1, nb, 16)
    sc = r[:, cols // 2:].copy().view(np.float16).astype(np.float32)
    idx = np.concatenate([codes & 15, codes >> 4], axis=2)
    kv = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
    return (kv[idx] * sc[:, :, None]).reshape(-1, cols)
