"""ctypes binding of libqe_moe.so (the C ABI in include/qe_moe.h).

The host side of the MoE block is the C ABI itself; this module only lets
Python drive it (tests, bench.py, __graft_entry__.smoke()).  Device memory is
handed over as raw pointers; torch tensors are accepted for convenience and
only their data_ptr() is used.  There is no fallback: if the shared library is
missing, LibraryMissing is raised.

The entry points mirror the reference engine's MoE call sites
(engine/qe.cpp:1957 Engine::moe_batched, :2466-2572 decode, :1653-1737
decode_multi<NT>): one context per GPU owning the flat expert arena.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqe_moe.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "qe_moe.h")

D = 2048
N_EXPERT = 256
K_USED = 8
FF_EXP = 512
ROUTER_ROWS = 257
EXPERT_BYTES = 1769472
SH_GU_BYTES = 1024 * 2176
SH_DN_BYTES = 2048 * 544

NPROF = 11
# ggml type ids of converter sources (QE_SRC_* in the header)
SRC_F32, SRC_F16, SRC_Q8_0, SRC_BF16 = 0, 1, 8, 30
QE_OK, QE_ERR_ARG, QE_ERR_HIP, QE_ERR_OOM, QE_ERR_STATE = 0, -1, -2, -3, -4
QE_MOE_DISPATCH_NOALLOC_T_MAX = 16384  # include/qe_moe.h
QE_MOE_T_MAX = 65536  # include/qe_moe.h: the largest t_max of a context


class LibraryMissing(RuntimeError):
    pass


class QeError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"qe_moe error {code}: {msg}")
        self.code = code


_lib = None


def header_symbols(path: str = HEADER) -> list[str]:
    """Names of every function the public header declares."""
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(qe_moe_\w+)\s*\(", txt)) - {"QE_MOE_NPROF"})


def load(path: str = LIB_PATH):
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise LibraryMissing(f"{path} not built (run __graft_entry__.build() or make -C qe-qwen36-b50_amd)")
    lib = ctypes.CDLL(path)
    vp, i32, i64, u64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t
    sig = {
        "qe_moe_create": (i32, [i32, i32, i32, ctypes.POINTER(vp)]),
        "qe_moe_destroy": (i32, [vp]),
        "qe_moe_expert_bytes": (sz, []),
        "qe_moe_upload_experts": (i32, [vp, i32, i32, i32, vp, i32, vp]),
        "qe_moe_set_dense": (i32, [vp, i32, vp, vp, vp, vp, vp, i32, vp]),
        "qe_moe_forward": (i32, [vp, i32, vp, vp, i32, vp]),
        "qe_moe_forward_normed": (i32, [vp, i32, vp, vp, i32, vp]),
        "qe_moe_forward_norm": (i32, [vp, i32, vp, vp, i32, vp, vp, vp]),
        "qe_moe_forward_stack": (i32, [vp, i32, i32, vp, vp, i32, vp]),
        "qe_moe_get_routing": (i32, [vp, i32, vp, vp, vp, vp, vp, vp, vp]),
        "qe_moe_get_logits": (i32, [vp, i32, vp, vp]),
        "qe_moe_dispatch": (i32, [vp, vp, i32, vp]),
        "qe_moe_arena_ptr": (i32, [vp, i32, ctypes.POINTER(vp)]),
        "qe_moe_load_pack": (i32, [vp, ctypes.c_char_p, i32, i32, i32, vp]),
        "qe_moe_synth_layer": (i32, [vp, i32, u64, vp, vp]),
        "qe_moe_synth_x": (i32, [u64, i32, vp, i64, vp]),
        "qe_moe_synth_zipf_bias": (i32, [u64, i32, ctypes.c_double, vp]),
        "qe_moe_last_error": (ctypes.c_char_p, []),
        "qe_moe_profile": (i32, [vp, i32]),
        "qe_moe_profile_read": (i32, [vp, vp, vp, i32]),
        "qe_moe_profile_name": (ctypes.c_char_p, [i32]),
        "qe_moe_nl4_quantize_rows": (i32, [vp, i32, i64, i32, vp, vp]),
        "qe_moe_convert_experts": (i32, [vp, i32, vp, vp, vp, i32, vp]),
        "qe_moe_check": (i32, [vp, vp]),
        "qe_moe_dispatch_noalloc": (i32, [vp, i32, vp, vp, vp]),
        "qe_moe_debug_set_epoch": (i32, [vp, ctypes.c_uint32, vp]),
        "qe_moe_debug_set_spin_cap": (i32, [vp, i32]),
        "qe_moe_debug_fused_wait_extra": (i32, [vp, i32]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    _lib = lib
    return lib


def _ptr(x):
    """Raw address of a torch tensor / numpy array / int / None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if isinstance(x, np.ndarray):
        assert x.flags["C_CONTIGUOUS"]
        return x.ctypes.data
    raise TypeError(type(x))


def _check(rc):
    if rc != QE_OK:
        raise QeError(rc, _lib.qe_moe_last_error().decode())


def _stream(s):
    if s is None:
        return None
    if hasattr(s, "cuda_stream"):
        return s.cuda_stream
    return s


class MoE:
    """One context on one GPU: arena of n_layers x 256 experts, scratch for t_max tokens."""

    def __init__(self, n_layers: int, t_max: int, device: int = 0):
        lib = load()
        h = ctypes.c_void_p()
        _check(lib.qe_moe_create(device, n_layers, t_max, ctypes.byref(h)))
        self.h, self.n_layers, self.t_max, self.device = h, n_layers, t_max, device

    def close(self):
        if self.h:
            _lib.qe_moe_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- weights --
    def synth_layer(self, layer, seed, bias: np.ndarray | None = None, stream=None):
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        _check(_lib.qe_moe_synth_layer(self.h, layer, seed, _ptr(b), _stream(stream)))

    def upload_experts(self, layer, first, blobs, on_device=False, stream=None):
        n = (blobs.nbytes if isinstance(blobs, np.ndarray) else blobs.numel() * blobs.element_size()) // EXPERT_BYTES
        _check(_lib.qe_moe_upload_experts(self.h, layer, first, n, _ptr(blobs), int(on_device), _stream(stream)))

    def set_dense(self, layer, post_norm=None, router=None, bias=None, sh_gu=None, sh_down=None, on_device=False,
                  stream=None):
        _check(_lib.qe_moe_set_dense(self.h, layer, _ptr(post_norm), _ptr(router), _ptr(bias), _ptr(sh_gu),
                                     _ptr(sh_down), int(on_device), _stream(stream)))

    def load_pack(self, path, pack_first, first_layer, n_layers, stream=None):
        _check(_lib.qe_moe_load_pack(self.h, str(path).encode(), pack_first, first_layer, n_layers, _stream(stream)))

    def convert_experts(self, layer, gate, up, down, src_type, stream=None):
        """Quantize blk.N.ffn_{gate,up,down}_exps (device tensors of ggml type src_type) into the layer's arena."""
        _check(_lib.qe_moe_convert_experts(self.h, layer, _ptr(gate), _ptr(up), _ptr(down), src_type,
                                           _stream(stream)))

    def arena_ptr(self, layer) -> int:
        p = ctypes.c_void_p()
        _check(_lib.qe_moe_arena_ptr(self.h, layer, ctypes.byref(p)))
        return p.value

    # -- compute --
    def forward(self, layer, x2, out, T, stream=None):
        _check(_lib.qe_moe_forward(self.h, layer, _ptr(x2), _ptr(out), T, _stream(stream)))

    def forward_norm(self, layer, x2, out, T, next_norm, xn, stream=None):
        """out = x2 + MoE(RMSNorm(x2)); xn = RMSNorm(out) * next_norm (the next block's input)."""
        _check(_lib.qe_moe_forward_norm(self.h, layer, _ptr(x2), _ptr(out), T, _ptr(next_norm), _ptr(xn),
                                        _stream(stream)))

    def forward_normed(self, layer, xn, out, T, stream=None):
        _check(_lib.qe_moe_forward_normed(self.h, layer, _ptr(xn), _ptr(out), T, _stream(stream)))

    def forward_stack(self, first, n, x_in, x_out, T, stream=None):
        _check(_lib.qe_moe_forward_stack(self.h, first, n, _ptr(x_in), _ptr(x_out), T, _stream(stream)))

    def routing(self, T, stream=None):
        ids = np.empty((T, K_USED), np.int32)
        wts = np.empty((T, K_USED), np.float32)
        shg = np.empty(T, np.float32)
        off = np.empty(N_EXPERT + 1, np.int32)
        pairs = np.empty(T * K_USED, np.int32)
        sd = np.empty((T, D), np.float32)
        _check(_lib.qe_moe_get_routing(self.h, T, _ptr(ids), _ptr(wts), _ptr(shg), _ptr(off), _ptr(pairs), _ptr(sd),
                                       _stream(stream)))
        return dict(ids=ids, wts=wts, shg=shg, off=off, pairs=pairs, sd=sd)

    def check(self, stream=None):
        """Synchronise `stream`; raise QeError if a decode launch timed out in an exchange poll, or a fused
        prefill launch in a down workgroup's wait."""
        _check(_lib.qe_moe_check(self.h, _stream(stream)))

    def debug_set_epoch(self, epoch, stream=None):
        _check(_lib.qe_moe_debug_set_epoch(self.h, epoch, _stream(stream)))

    def debug_set_spin_cap(self, cap):
        _check(_lib.qe_moe_debug_set_spin_cap(self.h, cap))

    def debug_fused_wait_extra(self, extra):
        _check(_lib.qe_moe_debug_fused_wait_extra(self.h, extra))

    def dispatch(self, ids_dev, T, stream=None):
        _check(_lib.qe_moe_dispatch(self.h, _ptr(ids_dev), T, _stream(stream)))

    def profile(self, enable: bool):
        _check(_lib.qe_moe_profile(self.h, int(enable)))

    def profile_read(self) -> dict:
        ms = np.zeros(NPROF, np.float64)
        n = np.zeros(NPROF, np.int32)
        _check(_lib.qe_moe_profile_read(self.h, _ptr(ms), _ptr(n), NPROF))
        return {_lib.qe_moe_profile_name(i).decode(): (float(ms[i]), int(n[i])) for i in range(NPROF) if n[i]}

    def logits(self, T, stream=None):
        lg = np.empty((T, ROUTER_ROWS), np.float32)
        _check(_lib.qe_moe_get_logits(self.h, T, _ptr(lg), _stream(stream)))
        return lg


def dispatch_noalloc(ids_dev, T, off_dev, pairs_dev, stream=None):
    """Context-free dispatch into caller buffers (no allocation; scratch in a static device array)."""
    load()
    _check(_lib.qe_moe_dispatch_noalloc(_ptr(ids_dev), T, _ptr(off_dev), _ptr(pairs_dev), _stream(stream)))


def synth_zipf_bias(seed, layer, s):
    """Host fp32[256] router bias -s * ln(rank) over a seeded permutation of the ranks (benchmark set-up)."""
    load()
    out = np.empty(N_EXPERT, np.float32)
    _check(_lib.qe_moe_synth_zipf_bias(seed, layer, float(s), _ptr(out)))
    return out


def synth_x(seed, inst, dev_out, n, stream=None):
    load()
    _check(_lib.qe_moe_synth_x(seed, inst, _ptr(dev_out), n, _stream(stream)))


def nl4_quantize_rows(src, src_type, rows, cols, dst, stream=None):
    """rows x cols weights of ggml type src_type (device) -> NL4 rows in dst (device), on the current device."""
    load()
    _check(_lib.qe_moe_nl4_quantize_rows(_ptr(src), src_type, rows, cols, _ptr(dst), _stream(stream)))
