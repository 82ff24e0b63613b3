"""Pre-swizzled AR GGUF: the layer projections stored in the matrix-core operand order.

The reference's exporter (tools/export_gguf/convert_ar.py:76-130) and quantiser
(tools/quantize_gguf.cpp) write each Q8_0 projection as ggml blocks `{fp16 d; int8 q[32]}`, row
after row. That file stays the contract: the library loads it as it is and reorders the quants on
the device. This tool writes an optional second form of the same model, in which every layer
projection `X` ([n][k], Q8_0, n % 32 == 0) is replaced by two tensors of standard GGUF types:

    X.qt  I8  [k, n]     the quants in the Q8_TILED order: per 32-row tile and block a 1 KB
                         chunk whose bytes [16 L, 16 L + 16), L = 32 h + i, are quants
                         [16 h, 16 h + 16) of row i of the tile
    X.dt  F16 [k/32, n]  the block scales in the same order: per tile and block, row i's scale

and the key `gsvk.q8_layout` = 1 is added. The loader copies these to the device unchanged and
derives the GEMV's sliced copy from them, so no quant is reordered on the host. Every other
tensor and key is copied byte for byte, in order, and `--back` restores the block form: a file
whose tensors are each padded to the alignment (as gguf-py writes them) comes back byte-identical.

    python gsv.cpp_amd/gguf_tiled.py ar.gguf ar.tiled.gguf
    python gsv.cpp_amd/gguf_tiled.py --back ar.tiled.gguf ar.gguf
"""
from __future__ import annotations

import argparse
import re
import struct
import sys

import numpy as np

GGML_F32, GGML_F16, GGML_Q8_0, GGML_I8 = 0, 1, 8, 24
KEY_LAYOUT = "gsvk.q8_layout"
LAYOUT_TILED32 = 1
_PROJ = re.compile(r"^transformer\.block\d+\.(qkv_w|out_w|ffn1_w|ffn2_w)$")

# GGUF value types: fixed sizes of the scalar ones
_T_STR, _T_ARR = 8, 9
_SCALAR = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


class Gguf:
    """A GGUF file as its parts: version, key/value entries (raw bytes each), alignment, tensors
    (name, ne in ggml order, type, data bytes) in directory order."""

    def __init__(self, version, kvs, alignment, tensors):
        self.version = version
        self.kvs = kvs              # list of (key, raw bytes of the whole entry)
        self.alignment = alignment
        self.tensors = tensors      # list of dict(name, ne, type, data)


def _tensor_bytes(ttype: int, ne) -> int:
    n = int(np.prod(ne))
    if ttype == GGML_F32:
        return 4 * n
    if ttype == GGML_F16:
        return 2 * n
    if ttype == GGML_Q8_0:
        return n // 32 * 34
    if ttype == GGML_I8:
        return n
    raise ValueError(f"tensor type {ttype} not handled")


def read(path: str) -> Gguf:
    buf = open(path, "rb").read()
    if buf[:4] != b"GGUF":
        raise ValueError(f"{path}: not a GGUF file")
    version, n_t, n_kv = struct.unpack_from("<IQQ", buf, 4)
    pos = 24

    def rd_str(p):
        n = struct.unpack_from("<Q", buf, p)[0]
        return buf[p + 8:p + 8 + n].decode(), p + 8 + n

    def skip_val(t, p):
        if t == _T_STR:
            return p + 8 + struct.unpack_from("<Q", buf, p)[0]
        if t == _T_ARR:
            et, cnt = struct.unpack_from("<IQ", buf, p)
            p += 12
            if et in _SCALAR:
                return p + _SCALAR[et] * cnt
            for _ in range(cnt):
                p = skip_val(et, p)
            return p
        return p + _SCALAR[t]

    kvs, alignment = [], 32
    for _ in range(n_kv):
        start = pos
        key, pos = rd_str(pos)
        t = struct.unpack_from("<I", buf, pos)[0]
        if key == "general.alignment":
            alignment = struct.unpack_from("<I", buf, pos + 4)[0]
        pos = skip_val(t, pos + 4)
        kvs.append((key, buf[start:pos]))
    infos = []
    for _ in range(n_t):
        name, pos = rd_str(pos)
        nd = struct.unpack_from("<I", buf, pos)[0]
        ne = list(struct.unpack_from(f"<{nd}Q", buf, pos + 4))
        pos += 4 + 8 * nd
        ttype, off = struct.unpack_from("<IQ", buf, pos)
        pos += 12
        infos.append((name, ne, ttype, off))
    data0 = (pos + alignment - 1) // alignment * alignment
    tensors = []
    for name, ne, ttype, off in infos:
        nb = _tensor_bytes(ttype, ne)
        a = data0 + off
        if a + nb > len(buf):
            raise ValueError(f"{path}: tensor {name} extends past the end of the file")
        tensors.append({"name": name, "ne": ne, "type": ttype, "data": buf[a:a + nb]})
    return Gguf(version, kvs, alignment, tensors)


def write(path: str, g: Gguf) -> None:
    def s(x: str) -> bytes:
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    A = g.alignment
    head = bytearray(b"GGUF" + struct.pack("<IQQ", g.version, len(g.tensors), len(g.kvs)))
    for _, raw in g.kvs:
        head += raw
    off = 0
    for t in g.tensors:
        head += s(t["name"]) + struct.pack("<I", len(t["ne"])) + struct.pack(f"<{len(t['ne'])}Q", *t["ne"])
        head += struct.pack("<IQ", t["type"], off)
        off += (len(t["data"]) + A - 1) // A * A
    head += b"\0" * ((-len(head)) % A)
    with open(path, "wb") as f:
        f.write(head)
        for t in g.tensors:
            f.write(t["data"])
            f.write(b"\0" * ((-len(t["data"])) % A))


def to_tiled(blocks: bytes, n: int, k: int) -> tuple[bytes, bytes]:
    """Q8_0 blocks of an [n][k] matrix -> (quants, scales) in the Q8_TILED order."""
    nblk, nt = k // 32, n // 32
    b = np.frombuffer(blocks, np.uint8).reshape(n, nblk, 34)
    q = b[:, :, 2:]                                   # [n][nblk][32]
    d = b[:, :, 0:2].copy().view(np.uint16)[:, :, 0]  # [n][nblk]
    # tile T, row i, block, half h, byte c -> [T][block][h][i][c]
    qt = q.reshape(nt, 32, nblk, 2, 16).transpose(0, 2, 3, 1, 4)
    dt = d.reshape(nt, 32, nblk).transpose(0, 2, 1)
    return np.ascontiguousarray(qt).tobytes(), np.ascontiguousarray(dt).astype("<u2").tobytes()


def from_tiled(qt: bytes, dt: bytes, n: int, k: int) -> bytes:
    """The inverse of to_tiled: the Q8_0 blocks of the [n][k] matrix."""
    nblk, nt = k // 32, n // 32
    q = np.frombuffer(qt, np.uint8).reshape(nt, nblk, 2, 32, 16).transpose(0, 3, 1, 2, 4).reshape(n, nblk, 32)
    d = np.frombuffer(dt, "<u2").reshape(nt, nblk, 32).transpose(0, 2, 1).reshape(n, nblk)
    out = np.empty((n, nblk, 34), np.uint8)
    out[:, :, 0:2] = d.astype("<u2")[:, :, None].view(np.uint8).reshape(n, nblk, 2)
    out[:, :, 2:] = q
    return out.tobytes()


def _u32_entry(key: str, v: int) -> bytes:
    b = key.encode()
    return struct.pack("<Q", len(b)) + b + struct.pack("<II", 4, v)


def tile(g: Gguf) -> Gguf:
    if any(k == KEY_LAYOUT for k, _ in g.kvs):
        raise ValueError("the file is already pre-swizzled")
    tensors = []
    for t in g.tensors:
        k, n = (t["ne"] + [1])[:2]
        if _PROJ.match(t["name"]) and t["type"] == GGML_Q8_0 and len(t["ne"]) == 2 and n % 32 == 0 and k % 32 == 0:
            qt, dt = to_tiled(t["data"], n, k)
            tensors.append({"name": t["name"] + ".qt", "ne": [k, n], "type": GGML_I8, "data": qt})
            tensors.append({"name": t["name"] + ".dt", "ne": [k // 32, n], "type": GGML_F16, "data": dt})
        else:
            tensors.append(t)
    return Gguf(g.version, g.kvs + [(KEY_LAYOUT, _u32_entry(KEY_LAYOUT, LAYOUT_TILED32))], g.alignment, tensors)


def untile(g: Gguf) -> Gguf:
    kvs = [(k, raw) for k, raw in g.kvs if k != KEY_LAYOUT]
    if len(kvs) == len(g.kvs):
        raise ValueError("the file is not pre-swizzled")
    tensors, i = [], 0
    while i < len(g.tensors):
        t = g.tensors[i]
        if t["name"].endswith(".qt"):
            base = t["name"][:-3]
            td = g.tensors[i + 1] if i + 1 < len(g.tensors) else None
            if td is None or td["name"] != base + ".dt":
                raise ValueError(f"{t['name']} is not followed by {base}.dt")
            k, n = t["ne"]
            tensors.append({"name": base, "ne": [k, n], "type": GGML_Q8_0,
                            "data": from_tiled(t["data"], td["data"], n, k)})
            i += 2
        else:
            tensors.append(t)
            i += 1
    return Gguf(g.version, kvs, g.alignment, tensors)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("src")
    ap.add_argument("dst")
    ap.add_argument("--back", action="store_true", help="restore the Q8_0 block form")
    a = ap.parse_args(argv)
    g = read(a.src)
    write(a.dst, untile(g) if a.back else tile(g))
    return 0


if __name__ == "__main__":
    sys.exit(main())
