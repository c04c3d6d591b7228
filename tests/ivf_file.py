"""Reader for vdb's VDBIVFP1 index file (test helper).

Layout (src/index/quant/ivf_pq.cc:236-249, src/index/index.cc:38-56): 8-byte magic, body,
then the CRC32C of everything before the 4-byte footer.  Body: u64 rows, u32 padded_dim,
u32 nlist, nlist x padded_dim fp32 coarse centroids, the product quantizer (u32 dim, u32 m,
m x 256 x dim/m fp32, src/index/quant/pq.cc:75-80), then per list: u64 size, size u32 ids,
size x m code bytes.
"""
import struct

import numpy as np


def parse_ivfpq(blob):
    blob = bytes(blob)
    assert blob[:8] == b"VDBIVFP1", blob[:8]
    p = 8
    rows, pd, nlist = struct.unpack_from("<QII", blob, p)
    p += 16
    coarse = np.frombuffer(blob, np.float32, nlist * pd, p).reshape(nlist, pd).copy()
    p += nlist * pd * 4
    dim, m = struct.unpack_from("<II", blob, p)
    p += 8
    dsub = dim // m
    cen = np.frombuffer(blob, np.float32, m * 256 * dsub, p).copy()
    p += m * 256 * dsub * 4
    off = [0]
    ids, codes = [], []
    for _ in range(nlist):
        (sz,) = struct.unpack_from("<Q", blob, p)
        p += 8
        ids.append(np.frombuffer(blob, np.uint32, sz, p))
        p += sz * 4
        codes.append(np.frombuffer(blob, np.uint8, sz * m, p))
        p += sz * m
        off.append(off[-1] + sz)
    assert p == len(blob) - 4, (p, len(blob))
    (crc,) = struct.unpack_from("<I", blob, p)
    return {
        "rows": rows, "pd": pd, "nlist": nlist, "dim": dim, "m": m, "coarse": coarse,
        "pq_centroids": cen, "list_off": np.array(off, np.uint64),
        "list_ids": np.ascontiguousarray(np.concatenate(ids) if ids else np.zeros(0, np.uint32)),
        "list_codes": np.ascontiguousarray(
            np.concatenate(codes) if codes else np.zeros(0, np.uint8)),
        "crc": crc, "crc_covered": blob[:-4],
    }
