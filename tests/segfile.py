"""Writers of vdb's segment files for the tests, field by field from the reference's layout:

  vectors.f32   src/storage/segment_writer.cc:58-75 (4 KiB header, then padded rows)
  blob files    src/storage/file_format.cc:8-18 ([magic 8][u32 1][u32 CRC32C][u64 len][payload])
  roaring       the portable serialization of a 32-bit roaring bitmap (RoaringFormatSpec),
                which Roaring::write(buf, true) emits (segment_writer.cc:29-39)

CRC32C comes from the oracle (its own restatement, pinned by known answers), not from the
library under test.
"""
import struct

import numpy as np

from oracle_lib import load_oracle

_OR = None


def crc32c(data):
    global _OR
    if _OR is None:
        _OR = load_oracle()
    data = bytes(data)
    return int(_OR.lib.or_crc32c(0, data, len(data)))


def vectors_file(rows, dim, metric, lsn=7):
    """vectors.f32 for padded rows (n, pd)."""
    rows = np.ascontiguousarray(rows, np.float32)
    n, pd = rows.shape
    data = rows.tobytes()
    h = bytearray(4096)
    h[0:8] = b"VDBSEG01"
    struct.pack_into("<IIQIIQQI", h, 8, 1, metric, n, dim, pd, 4096, len(data), crc32c(data))
    struct.pack_into("<QQ", h, 56, 0, lsn)
    struct.pack_into("<I", h, 4092, crc32c(bytes(h[:4092])))
    return bytes(h) + data


def blob(magic, payload, version=1):
    payload = bytes(payload)
    return (magic.encode()[:8].ljust(8, b"\0") + struct.pack("<IIQ", version, crc32c(payload),
                                                             len(payload)) + payload)


# ---- portable roaring bitmaps, one container description at a time
#   ("array", key, [u16 values]), ("bitmap", key, words[1024] uint64), ("run", key, [(start, len-1)])

def _card(c):
    kind, _, body = c
    if kind == "array":
        return len(body)
    if kind == "bitmap":
        return int(sum(bin(int(w)).count("1") for w in body))
    return sum(length + 1 for _, length in body)


def roaring(containers, runs_cookie=None):
    """The portable stream of containers (ascending keys).  runs_cookie: None = the run
    cookie exactly when some container is a run (as CRoaring writes), else forced."""
    has_run = any(c[0] == "run" for c in containers) if runs_cookie is None else runs_cookie
    n = len(containers)
    out = bytearray()
    if has_run:
        out += struct.pack("<I", 12347 | ((n - 1) << 16))
        flags = bytearray((n + 7) // 8)
        for i, c in enumerate(containers):
            if c[0] == "run":
                flags[i >> 3] |= 1 << (i & 7)
        out += flags
    else:
        out += struct.pack("<II", 12346, n)
    for kind, key, body in containers:
        out += struct.pack("<HH", key, _card((kind, key, body)) - 1)
    bodies = []
    for kind, key, body in containers:
        if kind == "array":
            bodies.append(struct.pack(f"<{len(body)}H", *body))
        elif kind == "bitmap":
            bodies.append(np.asarray(body, np.uint64).tobytes())
        else:
            bodies.append(struct.pack("<H", len(body)) +
                          b"".join(struct.pack("<HH", s, ln) for s, ln in body))
    if not has_run or n >= 4:
        off = len(out) + 4 * n
        for b in bodies:
            out += struct.pack("<I", off)
            off += len(b)
    for b in bodies:
        out += b
    return bytes(out)


def dense_words(values, rows):
    w = np.zeros((rows + 63) // 64, np.uint64)
    v = np.asarray(sorted(set(values)), np.int64)
    np.bitwise_or.at(w, v // 64, np.uint64(1) << (v % 64).astype(np.uint64))
    return w
