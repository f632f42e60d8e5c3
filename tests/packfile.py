"""Writer of weight packs in the reference engine's file layout (engine/pack.h:45-54):
a 24-byte header {"QE36PK01", n_entries, pad, table_off}, the tensor bytes, then a
table of 128-byte entries {name[96], fmt, rows, cols, n, off, bytes}.  Test
infrastructure: builds small synthetic packs for the loader's parity and error tests.
"""
import struct

import numpy as np

F_F32, F_Q8, F_Q6, F_NL4 = 0, 1, 2, 3


def write_pack(path, entries, magic=b"QE36PK01"):
    """entries: list of (name, fmt, rows, cols, n, ndarray); data is written as raw bytes."""
    with open(path, "wb") as f:
        f.write(b"\0" * 24)
        table = []
        for name, fmt, rows, cols, n, arr in entries:
            off = f.tell()
            raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
            f.write(raw.tobytes())
            table.append((name, fmt, rows, cols, n, off, raw.size))
        table_off = f.tell()
        for name, fmt, rows, cols, n, off, nbytes in table:
            f.write(struct.pack("<96s4I2Q", name.encode(), fmt, rows, cols, n, off, nbytes))
        f.seek(0)
        f.write(struct.pack("<8s2IQ", magic, len(table), 0, table_off))


def q8_rows(rng, rows, cols, scale=0.0005):
    """Q8 rows: cols int8 then cols/32 fp16 scales (engine/pack.h:24)."""
    q = rng.integers(-127, 128, (rows, cols), dtype=np.int8).view(np.uint8)
    s = np.full((rows, cols // 32), scale, np.float16).view(np.uint8).reshape(rows, -1)
    return np.concatenate([q, s], axis=1)


def nl4_rows(rng, lead, rows, cols):
    """NL4 rows: cols/2 code bytes then cols/32 fp16 scales |N(0,1)| * 0.02 (engine/pack.h:27)."""
    q = rng.integers(0, 256, lead + (rows, cols // 2), dtype=np.uint8)
    s = (np.abs(rng.standard_normal(lead + (rows, cols // 32))) * 0.02).astype(np.float16)
    return np.concatenate([q, s.view(np.uint8)], axis=-1)


def synth_moe_tensors(seed, D=2048, FF=512, NE=256):
    """One layer's MoE tensors, the way the engine's pack names them."""
    rng = np.random.default_rng(seed)
    gu = nl4_rows(rng, (NE,), 2 * FF, D)          # gate rows then up rows
    dn = nl4_rows(rng, (NE,), D, FF)
    experts = np.concatenate([gu.reshape(NE, -1), dn.reshape(NE, -1)], axis=1)
    return dict(
        post_norm=(0.5 + rng.random(D)).astype(np.float32),
        router=(rng.standard_normal((NE, D)) * 0.02).astype(np.float32),
        sh_gate=(rng.standard_normal(D) * 0.02).astype(np.float32),
        sh_gate_proj=q8_rows(rng, FF, D),
        sh_up=q8_rows(rng, FF, D),
        sh_down=q8_rows(rng, D, FF),
        experts=experts,
    )


def pack_entries(layer, t, fmt_override=None):
    pre = f"blk.{layer}."
    fo = fmt_override or {}
    return [
        (pre + "post_norm", fo.get("post_norm", F_F32), 1, 2048, 1, t["post_norm"]),
        (pre + "router", F_F32, 256, 2048, 1, t["router"]),
        (pre + "sh_gate", F_F32, 1, 2048, 1, t["sh_gate"]),
        (pre + "sh_gate_proj", F_Q8, 512, 2048, 1, t["sh_gate_proj"]),
        (pre + "sh_up", fo.get("sh_up", F_Q8), 512, 2048, 1, t["sh_up"]),
        (pre + "sh_down", F_Q8, 2048, 512, 1, t["sh_down"]),
        (pre + "experts", F_NL4, 3072, 2048, 256, t["experts"]),
    ]
