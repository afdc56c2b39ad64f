"""Writes safetensors shards for the store tests (test infrastructure).

A shard is [8-byte little-endian header length][JSON header][data], the header mapping
each tensor name to {"dtype", "shape", "data_offsets"} with offsets relative to the end
of the header.  The writer keeps the order it is given, so tests can lay an expert's six
tensors out as one run or scatter them.
"""
import json
import struct

import numpy as np

EXPERT = "language_model.model.layers.{l}.block_sparse_moe.experts.{e}.w{m}.{k}"


def expert_name(layer, expert, m, kind):
    """m: 1 gate, 2 down, 3 up; kind: 'weight_packed' or 'weight_scale'."""
    return EXPERT.format(l=layer, e=expert, m=m, k=kind)


def write_shard(path, tensors, metadata=None, pad=0):
    """tensors: list of (name, dtype string, shape, raw bytes); returns {name: (abs offset,
    nbytes)} as laid out.  pad: spaces appended to the header (alignment padding)."""
    hdr = {}
    if metadata is not None:
        hdr["__metadata__"] = metadata
    off = 0
    for name, dt, shape, raw in tensors:
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    hb = json.dumps(hdr).encode() + b" " * pad
    where = {}
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for name, dt, shape, raw in tensors:
            where[name] = (f.tell(), len(raw))
            f.write(raw)
    return where


def expert_tensors(layer, expert, d):
    """The six tensors of an expert (d: p1,s1,p3,s3,p2,s2 arrays) in the released
    checkpoint's order: w1 packed, w1 scale, w2 packed, w2 scale, w3 packed, w3 scale."""
    out = []
    for m, (pk, sk) in ((1, ("p1", "s1")), (2, ("p2", "s2")), (3, ("p3", "s3"))):
        for kind, key in (("weight_packed", pk), ("weight_scale", sk)):
            a = np.ascontiguousarray(d[key], np.uint8)
            out.append((expert_name(layer, expert, m, kind), "U8", a.shape, a.tobytes()))
    return out


def run_bytes(d):
    """The expert's bytes in run order."""
    return b"".join(np.ascontiguousarray(d[k], np.uint8).tobytes()
                    for k in ("p1", "s1", "p2", "s2", "p3", "s3"))
