"""Segment files a search opens (Segment::Open, src/storage/segment_reader.cc:20-122): CRC32C,
blob files, delete sets (portable roaring bitmaps expanded to dense words), vectors.f32 and
HNSW-SQ8 index files.

The delete-set decoder has no reference-written stream to compare with (CRoaring is not in
the reference tree or this image), so it is pinned by streams spelled out byte by byte from the
portable format's published layout, by set identities (runs, arrays and bitmaps of the same set
decode alike; both cookies decode alike) and by the reference's own error rule (a row at or
past the segment's end is corruption, segment_reader.cc:111).  The HNSW-SQ8 loader is pinned
against files written by the reference's own HnswSq8Index::save (tests/golden/segment.npz).
"""
import os
import struct

import numpy as np
import pytest

import segfile
import vdbg

HERE = os.path.dirname(os.path.abspath(__file__))


def _words_to_set(w):
    bits = np.unpackbits(w.view(np.uint8), bitorder="little")
    return set(np.nonzero(bits)[0].tolist())


# ---------------------------------------------------------------- CRC32C and blobs (CPU)

def test_crc32c_known_answers():
    assert vdbg.crc32c(b"123456789") == 0xE3069283  # tests/distance_test.cc:94
    assert vdbg.crc32c(b"") == 0
    g = np.load(os.path.join(HERE, "golden", "misc.npz"))
    blob = g["crc_blob"].tobytes()
    assert vdbg.crc32c(blob) == g["crc"][2]
    # Extend(Value(a), b) == Value(a + b) (crc32c.h:9-10), at every alignment
    for cut in (0, 1, 3, 7, 8, 9, 500, 999):
        assert vdbg.crc32c(blob[cut:], vdbg.crc32c(blob[:cut])) == g["crc"][2]
    big = np.random.default_rng(1).integers(0, 256, 1 << 20).astype(np.uint8).tobytes()
    assert vdbg.crc32c(big) == segfile.crc32c(big)


def test_blob_decode():
    payload = bytes(range(200))
    b = segfile.blob("VDBIDS01", payload)
    assert vdbg.blob_payload(b, "VDBIDS01") == payload
    cases = [
        (b[:20], "file shorter than its header"),
        (b"VDBIDX01" + b[8:], "bad file magic"),
        (segfile.blob("VDBIDS01", payload, version=2), "unsupported file version"),
        (b + b"\0", "file length mismatch"),
        (b[:-1] + bytes([b[-1] ^ 1]), "file checksum mismatch"),
    ]
    for bad, msg in cases:
        with pytest.raises(vdbg.VdbgError) as e:
            vdbg.blob_payload(bad, "VDBIDS01")
        assert e.value.code == 5 and msg in str(e.value)


# ---------------------------------------------------------------- delete sets (CPU)

def test_roaring_spelled_out_no_runs():
    # {1, 5, 70000}: cookie 12346, two containers, keys 0 and 1, offsets 24 and 28
    stream = bytes.fromhex(
        "3a300000" "02000000"      # cookie, container count
        "0000" "0100" "0100" "0000"  # (key 0, card-1 1), (key 1, card-1 0)
        "18000000" "1c000000"      # offsets
        "0100" "0500"              # key 0: 1, 5
        "7011")                    # key 1: 0x1170 = 70000 - 65536
    words, n = vdbg.decode_deletes(segfile.blob("VDBDEL01", stream), 70001)
    assert n == 3 and _words_to_set(words) == {1, 5, 70000}


def test_roaring_spelled_out_runs():
    # {10..19, 100}: cookie 12347 | (1-1) << 16, run flags 0b1, one container, no offsets
    stream = bytes.fromhex(
        "3b300000" "01"            # cookie, run-container bitset
        "0000" "0a00"              # key 0, card-1 10
        "0200" "0a000900" "64000000")  # two runs: (10, +9), (100, +0)
    words, n = vdbg.decode_deletes(segfile.blob("VDBDEL01", stream), 128)
    assert n == 11 and _words_to_set(words) == set(range(10, 20)) | {100}


def test_roaring_empty():
    words, n = vdbg.decode_deletes(segfile.blob("VDBDEL01", segfile.roaring([])), 1000)
    assert n == 0 and not words.any()
    words, n = vdbg.decode_deletes(segfile.blob("VDBDEL01", segfile.roaring([])), 0)
    assert n == 0 and words.size == 0


@pytest.mark.parametrize("with_runs,runs_cookie", [(True, None), (False, True), (False, False)])
def test_roaring_every_container_kind(with_runs, runs_cookie):
    # four containers with a run (run cookie, offset header present), three without a run
    # under either cookie (the run cookie then has no offset header)
    rng = np.random.default_rng(7)
    evens = np.zeros(1024, np.uint64)
    evens[:] = np.uint64(0x5555555555555555)           # bitmap: every even low value
    arr = sorted(rng.choice(65536, 300, replace=False).tolist())
    cont = [("bitmap", 0, evens), ("array", 1, arr), ("array", 3, [0, 65535])]
    expect = set(range(0, 65536, 2)) | {65536 + v for v in arr} | {3 << 16, (3 << 16) | 65535}
    if with_runs:
        cont.insert(2, ("run", 2, [(0, 99), (1000, 0), (65000, 535)]))
        expect |= {(2 << 16) + v for v in list(range(100)) + [1000] + list(range(65000, 65536))}
    rows = (4 << 16) + 5
    words, n = vdbg.decode_deletes(segfile.blob("VDBDEL01", segfile.roaring(cont, runs_cookie)), rows)
    assert n == len(expect)
    assert _words_to_set(words) == expect


def test_roaring_same_set_two_ways():
    # a container's kind follows its cardinality (arrays hold at most 4096 values, bitmaps
    # more); a run container may hold either, and decodes to the same words
    small = list(range(100, 3000)) + [40000]
    large = list(range(100, 9000)) + [40000]
    cases = [(small, ("array", 0, small)), (large, ("bitmap", 0, segfile.dense_words(large, 65536)))]
    for vals, plain in cases:
        want = segfile.dense_words(vals, 65536)
        run = ("run", 0, [(100, vals[-2] - 100), (40000, 0)])
        for form in (plain, run):
            w, n = vdbg.decode_deletes(segfile.blob("VDBDEL01", segfile.roaring([form])), 65536)
            assert n == len(vals) and np.array_equal(w, want), form[0]


def test_roaring_bad_streams():
    def dec(stream, rows=100000):
        return vdbg.decode_deletes(segfile.blob("VDBDEL01", stream), rows)

    good = segfile.roaring([("array", 0, [1, 2, 3]), ("array", 1, [7])])
    for bad in [b"", b"\x3a\x30", struct.pack("<I", 12345) + good[4:], good[:-1], good[:10]]:
        with pytest.raises(vdbg.VdbgError) as e:
            dec(bad)
        assert e.value.code == 5 and "malformed roaring" in str(e.value)
    # a row at or past the segment's end (segment_reader.cc:111)
    with pytest.raises(vdbg.VdbgError) as e:
        dec(good, rows=65536 + 7)
    assert e.value.code == 5 and "out of range" in str(e.value)
    dec(good, rows=65536 + 8)
    with pytest.raises(vdbg.VdbgError):
        vdbg.decode_deletes(segfile.blob("VDBIDS01", good), 100000)  # wrong magic
    # a non-empty set against a zero-row segment
    with pytest.raises(vdbg.VdbgError):
        dec(good, rows=0)


def test_golden_hnsw_sq8_files_parse():
    # the fixture's files carry the reference's CRC32C footer and quantizer layout
    g = np.load(os.path.join(HERE, "golden", "segment.npz"))
    for tag in ("a", "b"):
        f = g[f"{tag}_file"].tobytes()
        assert f[:8] == b"VDBHSQ81"
        assert vdbg.crc32c(f[:-4]) == struct.unpack("<I", f[-4:])[0]
        n, d, p = struct.unpack_from("<QII", f, 8)
        rows = g[f"{tag}_rows"]
        assert (n, d, p) == (rows.shape[0], int(g[f"{tag}_dim"]), rows.shape[1])
        vmin = np.frombuffer(f, np.float32, p, 24)
        scale = np.frombuffer(f, np.float32, p, 24 + 4 * p)
        codes = np.frombuffer(f, np.uint8, n * p, 24 + 8 * p).reshape(n, p)
        assert np.array_equal(vmin.view(np.uint32), g[f"{tag}_vmin"].view(np.uint32))
        assert np.array_equal(scale.view(np.uint32), g[f"{tag}_scale"].view(np.uint32))
        assert np.array_equal(codes, g[f"{tag}_codes"])


# ---------------------------------------------------------------- on the GPU

@pytest.mark.gpu
@pytest.mark.parametrize("n,dim,metric", [(5000, 128, "l2"), (777, 40, "ip"), (0, 16, "l2")])
def test_open_vectors_searches_like_the_rows(ctx, oracle, n, dim, metric):
    print(f"open_vectors n={n} dim={dim} {metric}", flush=True)
    pd = vdbg.padded_dim(dim)
    rows = np.zeros((n, pd), np.float32)
    rows[:, :dim] = np.random.default_rng(n + dim).standard_normal((n, dim))
    f = segfile.vectors_file(rows, dim, vdbg.METRICS[metric])
    ds = vdbg.Dataset.open_vectors(ctx, f, dim, metric, rows=n)
    assert ds.n == n
    if n == 0:
        ds.close()
        return
    q = np.zeros((20, pd), np.float32)
    q[:, :dim] = np.random.default_rng(3).standard_normal((20, dim))
    gi, gd = ds.flat_search(q, 10)
    od, oi = oracle.flat_search(rows, q, 10, metric=metric)
    assert np.array_equal(gi, oi) and np.array_equal(gd.view(np.uint32), od.view(np.uint32))
    ds.close()


@pytest.mark.gpu
def test_open_vectors_rejects_what_segment_open_rejects(ctx):
    n, dim = 300, 40
    pd = vdbg.padded_dim(dim)
    rows = np.random.default_rng(5).standard_normal((n, pd)).astype(np.float32)
    rows[:, dim:] = 0
    f = bytearray(segfile.vectors_file(rows, dim, 0))

    def expect(data, msg, **kw):
        args = dict(dim=dim, metric="l2", rows=n)
        args.update(kw)
        with pytest.raises(vdbg.VdbgError) as e:
            vdbg.Dataset.open_vectors(ctx, bytes(data), **args)
        assert e.value.code == 5 and msg in str(e.value), str(e.value)

    expect(f[:4000], "shorter than its header")
    expect(b"VDBSEG02" + f[8:], "bad magic")
    g = bytearray(f)
    g[100] ^= 1
    expect(g, "header checksum mismatch")
    expect(f, "does not match the manifest", rows=n + 1)
    expect(f, "does not match the manifest", metric="ip")
    expect(f, "does not match the manifest", dim=41)
    expect(f[:-4], "does not match the manifest")
    g = bytearray(f)
    g[5000] ^= 1
    expect(g, "data checksum mismatch")
    vdbg.Dataset.open_vectors(ctx, bytes(g), dim, "l2", rows=n, verify_crc=False).close()
    vdbg.Dataset.open_vectors(ctx, bytes(f) + b"tail", dim, "l2").close()


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["a", "b"])
def test_sq8_load_reference_file(ctx, oracle, tag):
    # a VDBHSQ81 file from the reference's HnswSq8Index::save: the resident codes are the
    # file's, and the SQ8 scan matches the index created by encoding the rows
    g = np.load(os.path.join(HERE, "golden", "segment.npz"))
    rows, dim = g[f"{tag}_rows"], int(g[f"{tag}_dim"])
    metric = ["l2", "ip"][int(g[f"{tag}_metric"])]
    print(f"sq8_load {tag} n={rows.shape[0]} dim={dim} {metric}", flush=True)
    ds = vdbg.Dataset(ctx, rows, dim, metric)
    sq = vdbg.Sq8Index.load(ds, g[f"{tag}_file"].tobytes())
    assert np.array_equal(sq.codes(), g[f"{tag}_codes"])
    assert np.array_equal(sq.vmin.view(np.uint32), g[f"{tag}_vmin"].view(np.uint32))
    enc = vdbg.Sq8Index(ds)
    q = rows[::37].copy() + np.float32(0.25)
    for depth in (0, 30):
        li, ld = sq.search(q, 10, depth)
        ei, ed = enc.search(q, 10, depth)
        assert np.array_equal(li, ei) and np.array_equal(ld.view(np.uint32), ed.view(np.uint32))
    od, oi = oracle.sq8_search(rows, g[f"{tag}_codes"], g[f"{tag}_vmin"], g[f"{tag}_scale"], q,
                               10, 30, metric=metric)
    li, ld = sq.search(q, 10, 30)
    assert np.array_equal(li, oi) and np.array_equal(ld.view(np.uint32), od.view(np.uint32))
    ds.close()


@pytest.mark.gpu
def test_sq8_load_rejects_bad_files(ctx):
    g = np.load(os.path.join(HERE, "golden", "segment.npz"))
    rows, dim = g["a_rows"], int(g["a_dim"])
    f = g["a_file"].tobytes()
    ds = vdbg.Dataset(ctx, rows, dim)
    other = vdbg.Dataset(ctx, rows[:-1], dim)

    def expect(d, data, msg):
        with pytest.raises(vdbg.VdbgError) as e:
            vdbg.Sq8Index.load(d, data)
        assert e.value.code == 5 and msg in str(e.value), str(e.value)

    expect(ds, f[:11], "too short")
    expect(ds, f[:-1] + bytes([f[-1] ^ 1]), "checksum mismatch")
    body = b"VDBHNSW1" + f[8:-4]
    expect(ds, body + struct.pack("<I", vdbg.crc32c(body)), "not an hnsw-sq8 index file")
    expect(other, f, "does not match the segment")
    cut = f[:24 + 8 * 48 + 100]
    expect(ds, cut + struct.pack("<I", vdbg.crc32c(cut)), "truncated sq8 codes")
    ds.close()
    other.close()
