"""Extract a small routing-record fixture from the reference's phase0/statsA.bin.

statsA.bin is data the reference ships (routing records written by
phase0/expert_stats.cpp:41-50: int16 layer, int32 n_tok, n_tok*8 uint8
expert ids, token-major; read back by engine/qe.cpp:1136-1142).  The fixture
keeps a few real-skew id streams as dispatch inputs; the expected per-expert
offsets and stable permutation are computed here with numpy's stable argsort
(the textbook definition of the reference's counting sort,
engine/qe.cpp:1968-1976), independently of the oracle.

Run in the build container (the reference tree is not on the GPU box):
    python tests/golden/make_routing_fixture.py /root/reference/phase0/statsA.bin
"""
import struct
import sys
import os

import numpy as np


def read_records(path, max_records):
    out = []
    with open(path, "rb") as f:
        while len(out) < max_records:
            hdr = f.read(6)
            if len(hdr) < 6:
                break
            layer, nt = struct.unpack("<hi", hdr)
            ids = np.frombuffer(f.read(nt * 8), np.uint8).reshape(nt, 8)
            out.append((layer, ids))
    return out


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/phase0/statsA.bin"
    recs = read_records(src, 200)
    keep = {}
    for layer, ids in recs:
        # the first full 512-token ubatch of layers 0, 1 and 39, plus one short record
        if ids.shape[0] == 512 and layer in (0, 1, 39) and ("L%d" % layer) not in keep:
            keep["L%d" % layer] = ids
        if ids.shape[0] < 512 and "short" not in keep:
            keep["short"] = ids
    arrays = {}
    for name, ids in keep.items():
        flat = ids.astype(np.int32).reshape(-1)
        cnt = np.bincount(flat, minlength=256)
        off = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
        pairs = np.argsort(flat, kind="stable").astype(np.int32)
        arrays[name + "_ids"] = ids
        arrays[name + "_off"] = off
        arrays[name + "_pairs"] = pairs
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "routing_records.npz")
    np.savez_compressed(out, **arrays)
    print("wrote", out, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
