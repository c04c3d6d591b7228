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


def write_ivfpq(rows, pd, coarse, dim, m, pq_centroids, list_ids, list_codes):
    """A VDBIVFP1 file (the layout above) from per-list id/code arrays."""
    from oracle_lib import load_oracle

    body = bytearray(b"VDBIVFP1")
    body += struct.pack("<QII", rows, pd, len(list_ids))
    body += np.ascontiguousarray(coarse, np.float32).tobytes()
    body += struct.pack("<II", dim, m)
    body += np.ascontiguousarray(pq_centroids, np.float32).tobytes()
    for ids, codes in zip(list_ids, list_codes):
        body += struct.pack("<Q", len(ids))
        body += np.ascontiguousarray(ids, np.uint32).tobytes()
        body += np.ascontiguousarray(codes, np.uint8).tobytes()
    crc = load_oracle().lib.or_crc32c(0, bytes(body), len(body))
    body += struct.pack("<I", crc)
    return bytes(body)


def synth_ivfpq(base, dim, nlist, m, seed=0, metric="l2"):
    """A valid IVF-PQ index over `base` (n x pd) built with the oracle's own assignment and
    encoder: coarse centroids are strided rows, codebooks random residual sub-vectors.
    Search parity does not depend on how an index was trained, only on its contents."""
    from oracle_lib import KSET, load_oracle

    o = load_oracle()
    n, pd = base.shape
    rng = np.random.default_rng(seed)
    coarse = np.ascontiguousarray(base[np.linspace(0, n - 1, nlist).astype(np.int64)] +
                                  rng.normal(0, 0.01, (nlist, pd)).astype(np.float32) *
                                  (np.arange(pd) < dim))
    assign = np.empty(n, np.uint32)
    o.lib.or_assign_nearest(KSET["avx512"], np.ascontiguousarray(base), n, pd, pd, coarse, nlist,
                            assign, None, 8)
    resid = (base[:, :dim] - coarse[assign][:, :dim]).astype(np.float32)
    dsub = dim // m
    cen = np.empty((m, 256, dsub), np.float32)
    for j in range(m):
        pick = rng.choice(n, 256, replace=n < 256)
        cen[j] = resid[pick, j * dsub:(j + 1) * dsub]
    cen = np.ascontiguousarray(cen.ravel())
    codes = np.empty((n, m), np.uint8)
    for i in range(n):
        o.lib.or_pq_encode(cen, m, dsub, np.ascontiguousarray(resid[i]), codes[i])
    order = np.argsort(assign, kind="stable")
    bounds = np.searchsorted(assign[order], np.arange(nlist + 1))
    list_ids = [order[bounds[l]:bounds[l + 1]].astype(np.uint32) for l in range(nlist)]
    list_codes = [codes[ids] for ids in list_ids]
    return write_ivfpq(n, pd, coarse, dim, m, cen, list_ids, list_codes)


def parse_pqflat(blob):
    """A VDBPQFL1 file (src/index/quant/ivf_pq.cc:81-87): magic, u64 rows, the product
    quantizer (u32 dim, u32 m, m x 256 x dim/m fp32), rows x m code bytes, CRC32C footer."""
    blob = bytes(blob)
    assert blob[:8] == b"VDBPQFL1", blob[:8]
    rows, dim, m = struct.unpack_from("<QII", blob, 8)
    p = 24
    dsub = dim // m
    cen = np.frombuffer(blob, np.float32, m * 256 * dsub, p).copy()
    p += m * 256 * dsub * 4
    codes = np.frombuffer(blob, np.uint8, rows * m, p).reshape(rows, m).copy()
    p += rows * m
    assert p == len(blob) - 4, (p, len(blob))
    return {"rows": rows, "dim": dim, "m": m, "pq_centroids": cen, "codes": codes}
