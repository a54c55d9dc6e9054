#!/usr/bin/env python3
"""Write the reference tiny model as an int8 container (test input).

The engine (overhang engines/qwen.c:213-218) switches to its int8 "stream"
mode when expert 0's gate_proj of layer 0 is stored with dtype I8 (st.h:49-55
maps I8/U8 to its quantised code 3).  In that mode it reads each routed
expert as raw int8 rows plus a float32 per-row scale tensor "<name>.qs"
(qwen.c:428-452), and it makes int8 twins of the dense and GDN projections
itself at load (qwen.c:269-274, qw_make).  The container layout is that of
the reference converter (tools/convert_qwen.py:21-27, 66-71): routed expert
weights as row-wise int8 with scale s = max(|w_row|, 1e-12) / 127 and
q = round-half-even(w / s) clamped to [-128, 127]; every other tensor
unchanged.  This file restates that rule in numpy and writes the
safetensors file directly (8-byte little-endian header length, JSON header,
raw data), so it needs neither torch nor the safetensors package.

usage: make_int8_container.py SRC_DIR DST_DIR
"""
from __future__ import annotations

import json
import os
import re
import shutil
import struct
import sys

import numpy as np

EXPERT = re.compile(r"model\.layers\.\d+\.mlp\.experts\.\d+\.(gate_proj|up_proj|down_proj)\.weight$")
_DT = {"F32": np.float32, "I8": np.int8}


def read_safetensors(path: str) -> dict[str, np.ndarray]:
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        head = json.loads(f.read(n))
        base = 8 + n
        out = {}
        for name, t in head.items():
            if name == "__metadata__":
                continue
            if t["dtype"] not in _DT:
                raise ValueError(f"{name}: dtype {t['dtype']} not handled")
            a, b = t["data_offsets"]
            f.seek(base + a)
            out[name] = np.frombuffer(f.read(b - a), dtype=_DT[t["dtype"]]).reshape(t["shape"])
    return out


def write_safetensors(path: str, tensors: dict[str, np.ndarray]) -> None:
    head, off, blobs = {}, 0, []
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name])
        dt = {np.dtype(np.float32): "F32", np.dtype(np.int8): "I8"}[a.dtype]
        blobs.append(a.tobytes())
        head[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(blobs[-1])]}
        off += len(blobs[-1])
    head["__metadata__"] = {"format": "pt"}
    h = json.dumps(head, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for blob in blobs:
            f.write(blob)


def quantize_rows(w: np.ndarray):
    """Row-wise int8 with the converter's rule (tools/convert_qwen.py:23-27)."""
    w = w.astype(np.float32)
    s = (np.maximum(np.abs(w).max(axis=1), np.float32(1e-12)) / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.rint(w / s[:, None]), -128, 127).astype(np.int8)
    return q, s


def write_container(src: str, dst: str) -> None:
    os.makedirs(dst, exist_ok=True)
    for fn in os.listdir(src):
        if fn.endswith(".json"):
            shutil.copy2(os.path.join(src, fn), os.path.join(dst, fn))
    t = read_safetensors(os.path.join(src, "model.safetensors"))
    out = {}
    for name, w in t.items():
        if EXPERT.search(name):
            q, s = quantize_rows(w)
            out[name] = q
            out[name + ".qs"] = s
        else:
            out[name] = w
    write_safetensors(os.path.join(dst, "model.safetensors"), out)


if __name__ == "__main__":
    if len(sys.argv) != 3:
        sys.exit(__doc__)
    write_container(sys.argv[1], sys.argv[2])
