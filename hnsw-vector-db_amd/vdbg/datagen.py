"""Deterministic synthetic workloads for the search benchmarks and parity tests.

A counter-based generator (no std::*_distribution, no numpy Generator state): value i of
stream `seed` is mix(splitmix64(seed) + (i + 1) * golden), the SplitMix64 output function
applied to the i-th state of a SplitMix64 sequence seeded by `seed`.

  uniform01   (u64 >> 40) * 2^-24, an fp32-exact value in [0, 1)
  normal      Box-Muller in fp64 on pairs: u1 = ((u >> 11) + 1) * 2^-53 in (0, 1],
              u2 = (u >> 11) * 2^-53, z = sqrt(-2 ln u1) * (cos, sin)(2 pi u2)

Workloads (sizes as quoted for vdb's flat, SQ8 and IVF-PQ paths):
  uniform      rows U[0,1)^d                                     (100k x 128 in the bench)
  sift_like    1,000 centres U[0,64)^d, row = rint(centre + 12 N(0,1)) clipped to
               [0, 255]; integer-valued floats, most components near 0  (1M x 128)
  clustered_unit  centres N(0,1)^d, row = centre + sigma N(0,1), L2-normalised (cosine)
"""
import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z):
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def rand_u64(seed, start, count):
    with np.errstate(over="ignore"):
        key = _mix(np.array([seed], np.uint64) + GOLDEN)[0]
        i = np.arange(start, start + count, dtype=np.uint64)
        return _mix(key + (i + np.uint64(1)) * GOLDEN)


def uniform01(seed, start, count):
    return (rand_u64(seed, start, count) >> np.uint64(40)).astype(np.float32) * np.float32(
        2.0 ** -24)


def normal(seed, start, count):
    """count standard normals (fp64), values [start, start + count) of stream `seed`."""
    p0 = start // 2
    p1 = (start + count + 1) // 2
    u = rand_u64(seed, 2 * p0, 2 * (p1 - p0)).reshape(-1, 2)
    u1 = ((u[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (u[:, 1] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    z = np.empty(2 * len(r))
    z[0::2] = r * np.cos(t)
    z[1::2] = r * np.sin(t)
    off = start - 2 * p0
    return z[off:off + count]


def pad(x, pd):
    n, d = x.shape
    if pd == d:
        return np.ascontiguousarray(x, np.float32)
    out = np.zeros((n, pd), np.float32)
    out[:, :d] = x
    return out


def uniform_rows(n, dim, seed):
    return uniform01(seed, 0, n * dim).reshape(n, dim)


def sift_like(n, dim, seed, centres_seed=2001, n_centres=1000, sigma=12.0, block=1 << 16):
    """Rows from the SIFT-like mixture: integer-valued floats in [0, 255]."""
    cen = uniform01(centres_seed, 0, n_centres * dim).reshape(n_centres, dim) * np.float32(64)
    pick = (rand_u64(seed ^ 0x5BD1E995, 0, n) % np.uint64(n_centres)).astype(np.int64)
    out = np.empty((n, dim), np.float32)
    for b in range(0, n, block):
        e = min(n, b + block)
        z = normal(seed, b * dim, (e - b) * dim).reshape(e - b, dim)
        v = np.rint(cen[pick[b:e]].astype(np.float64) + sigma * z)
        out[b:e] = np.clip(v, 0.0, 255.0).astype(np.float32) + np.float32(0.0)
    return out


def clustered_unit(n, dim, seed, centres_seed, n_centres, sigma, block=1 << 15):
    """Gaussian mixture rows, each normalised like NormalizeVector (src/util/dataset.cc:33-41)."""
    cen = normal(centres_seed, 0, n_centres * dim).reshape(n_centres, dim)
    pick = (rand_u64(seed ^ 0x5BD1E995, 0, n) % np.uint64(n_centres)).astype(np.int64)
    out = np.empty((n, dim), np.float32)
    for b in range(0, n, block):
        e = min(n, b + block)
        z = normal(seed, b * dim, (e - b) * dim).reshape(e - b, dim)
        v = (cen[pick[b:e]] + sigma * z).astype(np.float32)
        out[b:e] = normalize_rows(v)
    return out


def normalize_rows(v):
    """Unit rows in NormalizeVector's manner (fp64 sum of squares, inv = float(1/sqrt), fp32
    multiply); the fp64 sum is taken in numpy's order, so a row can differ from
    NormalizeVector's in the last bit.  Test data only: the searches take rows as given."""
    v = np.asarray(v, np.float32)
    norm = np.einsum("ij,ij->i", v.astype(np.float64), v.astype(np.float64))
    ok = (norm > 0) & np.isfinite(norm)
    inv = np.where(ok, 1.0 / np.sqrt(np.where(ok, norm, 1.0)), 1.0).astype(np.float32)
    return (v * inv[:, None]).astype(np.float32)


# ---------------------------------------------------------------- device generation
#
# The same streams computed with torch on any device, for workloads too large to generate
# quickly on the host (5M x 384).  uint64 values are carried in int64 bit patterns: products
# wrap modulo 2^64 as unsigned ones do, right shifts are made logical by masking, and the
# unsigned remainder is taken on halves.  Integer outputs equal the numpy functions above;
# fp64 transcendental results may differ from numpy's in the last bits, so rows generated
# on a device are read back from it wherever a CPU baseline needs the same rows.

def _s64(v):
    return v - (1 << 64) if v >= 1 << 63 else v


_GOLDEN_S = _s64(0x9E3779B97F4A7C15)
_M1_S = _s64(0xBF58476D1CE4E5B9)
_M2_S = _s64(0x94D049BB133111EB)


def _srl(z, s):
    return (z >> s) & ((1 << (64 - s)) - 1)


def _mix_t(z):
    z = (z ^ _srl(z, 30)) * _M1_S
    z = (z ^ _srl(z, 27)) * _M2_S
    return z ^ _srl(z, 31)


def rand_u64_t(torch, seed, start, count, device):
    """rand_u64 as an int64 tensor of the same bits."""
    key = int(_mix(np.array([seed], np.uint64) + GOLDEN)[0])
    i = torch.arange(start + 1, start + count + 1, dtype=torch.int64, device=device)
    return _mix_t(_s64(key) + i * _GOLDEN_S)


def umod_t(u, n):
    """Unsigned remainder of int64-carried uint64 values by n (n < 2^31)."""
    return (2 * (_srl(u, 1) % n) + (u & 1)) % n


def normal_t(torch, seed, start, count, device):
    p0 = start // 2
    p1 = (start + count + 1) // 2
    u = rand_u64_t(torch, seed, 2 * p0, 2 * (p1 - p0), device).view(-1, 2)
    u1 = (_srl(u[:, 0], 11).to(torch.float64) + 1.0) * 2.0 ** -53
    u2 = _srl(u[:, 1], 11).to(torch.float64) * 2.0 ** -53
    r = torch.sqrt(-2.0 * torch.log(u1))
    t = 2.0 * np.pi * u2
    z = torch.stack([r * torch.cos(t), r * torch.sin(t)], dim=1).view(-1)
    off = start - 2 * p0
    return z[off:off + count]


def clustered_unit_t(torch, n, dim, seed, centres_seed, n_centres, sigma, device, start_row=0,
                     unit=True, block=1 << 16):
    """clustered_unit rows [start_row, start_row + n) of stream `seed` as an fp32 tensor on
    `device`; unit=False leaves them unnormalised (raw queries for PrepareQuery)."""
    cen = normal_t(torch, centres_seed, 0, n_centres * dim, device).view(n_centres, dim)
    pick = umod_t(rand_u64_t(torch, seed ^ 0x5BD1E995, start_row, n, device), n_centres)
    out = torch.empty((n, dim), dtype=torch.float32, device=device)
    for b in range(0, n, block):
        e = min(n, b + block)
        z = normal_t(torch, seed, (start_row + b) * dim, (e - b) * dim, device).view(e - b, dim)
        v = (cen[pick[b:e]] + sigma * z).to(torch.float32)
        if unit:
            v64 = v.to(torch.float64)
            norm = (v64 * v64).sum(dim=1)
            ok = (norm > 0) & torch.isfinite(norm)
            inv = torch.where(ok, 1.0 / torch.sqrt(torch.where(ok, norm, 1.0)),
                              torch.ones_like(norm)).to(torch.float32)
            v = v * inv[:, None]
        out[b:e] = v
    return out
