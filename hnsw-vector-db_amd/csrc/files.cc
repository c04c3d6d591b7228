// files.cc -- the on-disk formats a segment is opened from (host-only code).
//
// Segment::Open (src/storage/segment_reader.cc:20-122) reads, for the search path:
//   vectors.f32        4 KiB header + padded fp32 rows (segment.h:9-12, segment_writer.cc:58-75)
//   ids.u64, deletes-n.roar
//                      blob files: [magic 8][u32 version 1][u32 CRC32C of the payload]
//                      [u64 payload length][payload] (src/storage/file_format.h:3-4,
//                      file_format.cc:8-33)
//   index.<type>       magic + body + CRC32C footer (src/index/index.cc:38-56)
// The delete set's payload is a roaring bitmap in the portable serialization written by
// Roaring::write(buf, true) (segment_writer.cc:29-39) and read by Roaring::readSafe
// (segment_reader.cc:108-117).  CRoaring is not part of this build; the decoder below follows
// the published format (RoaringFormatSpec, as implemented by CRoaring 4.2.1's
// roaring_bitmap_portable_deserialize_safe) and expands the set straight into the dense
// words the device filters take.
#include <immintrin.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>

#include "../../include/vdbg.h"

namespace vdbg {

int SetError(int code, const std::string& msg);  // vdbg_api.hip

namespace {

// CRC32C (Castagnoli, reflected polynomial 0x82F63B78), the checksum of every vdb file
// (src/util/crc32c.h:9-16): byte-wise tables in software, the SSE4.2 crc32 instruction when
// the host has it.  Both give the same value for every input.
struct CrcTable {
  uint32_t t[256];
  CrcTable() {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int b = 0; b < 8; ++b) c = (c >> 1) ^ (0x82F63B78u & (0u - (c & 1u)));
      t[i] = c;
    }
  }
};

uint32_t ExtendTable(uint32_t crc, const uint8_t* p, size_t n) {
  static const CrcTable tab;  // thread-safe initialisation
  uint32_t c = ~crc;
  for (size_t i = 0; i < n; ++i) c = tab.t[(c ^ p[i]) & 0xffu] ^ (c >> 8);
  return ~c;
}

__attribute__((target("sse4.2"))) uint32_t ExtendSse42(uint32_t crc, const uint8_t* p, size_t n) {
  uint64_t c = ~crc;
  for (; n > 0 && (reinterpret_cast<uintptr_t>(p) & 7u) != 0; --n) c = _mm_crc32_u8(uint32_t(c), *p++);
  for (; n >= 8; n -= 8, p += 8) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    c = _mm_crc32_u64(c, v);
  }
  uint32_t c32 = uint32_t(c);
  for (; n > 0; --n) c32 = _mm_crc32_u8(c32, *p++);
  return ~c32;
}

bool HaveSse42() {
  static const bool have = [] {
    __builtin_cpu_init();
    return __builtin_cpu_supports("sse4.2") != 0;
  }();
  return have;
}

template <class T>
T Get(const uint8_t* p) {
  T v;
  std::memcpy(&v, p, sizeof(T));
  return v;
}

int Corrupt(const std::string& what) { return SetError(VDBG_CORRUPTION, what); }

}  // namespace

uint32_t Crc32cExtend(uint32_t crc, const void* data, size_t n) {
  const auto* p = static_cast<const uint8_t*>(data);
  return HaveSse42() ? ExtendSse42(crc, p, n) : ExtendTable(crc, p, n);
}

uint32_t Crc32c(const void* data, size_t n) { return Crc32cExtend(0, data, n); }

// Segment::Open's vectors.f32 checks (segment_reader.cc:37-55), in the same order and with
// the same messages.  On success *data points at the first row (byte 4096) and *rows holds
// the header's row count.
int CheckSegmentVectors(const void* file, size_t len, size_t dim, int metric, uint64_t expect_rows,
                        int verify_crc, const float** data, uint64_t* rows) {
  constexpr size_t kHeader = 4096;  // kSegmentHeaderSize (segment.h:33)
  const auto* h = static_cast<const uint8_t*>(file);
  if (len < kHeader) return Corrupt("vectors.f32: shorter than its header");
  if (std::memcmp(h, "VDBSEG01", 8) != 0) return Corrupt("vectors.f32: bad magic");
  if (Get<uint32_t>(h + kHeader - 4) != Crc32c(h, kHeader - 4))
    return Corrupt("vectors.f32: header checksum mismatch");
  const uint64_t n = Get<uint64_t>(h + 16);
  const uint64_t data_len = Get<uint64_t>(h + 40);
  const uint64_t pd = (uint64_t(dim) + 15) / 16 * 16;
  // the product is formed only once n is known small enough for it not to wrap
  const bool size_ok = n <= (~uint64_t(0) - kHeader) / (pd * 4 + 1) && data_len == n * pd * 4 &&
                       len - kHeader >= data_len;
  if (Get<uint32_t>(h + 8) != 1 || Get<uint32_t>(h + 12) != uint32_t(metric) ||
      (expect_rows != ~uint64_t(0) && n != expect_rows) || Get<uint32_t>(h + 24) != dim ||
      Get<uint32_t>(h + 28) != pd || Get<uint64_t>(h + 32) != kHeader || !size_ok)
    return Corrupt("vectors.f32: header does not match the manifest");
  if (verify_crc && Crc32c(h + kHeader, data_len) != Get<uint32_t>(h + 48))
    return Corrupt("vectors.f32: data checksum mismatch");
  *data = reinterpret_cast<const float*>(h + kHeader);
  *rows = n;
  return VDBG_OK;
}

}  // namespace vdbg

using vdbg::Corrupt;
using vdbg::Get;

extern "C" {

uint32_t vdbg_crc32c_extend(uint32_t crc, const void* data, size_t n) {
  return vdbg::Crc32cExtend(crc, data, n);
}

int vdbg_blob_decode(const void* file, size_t len, const char* magic, size_t* payload_offset,
                     size_t* payload_len) {
  if (file == nullptr && len > 0) return vdbg::SetError(VDBG_INVALID_ARGUMENT, "null file");
  if (magic == nullptr || payload_offset == nullptr || payload_len == nullptr)
    return vdbg::SetError(VDBG_INVALID_ARGUMENT, "null argument");
  const auto* p = static_cast<const uint8_t*>(file);
  const size_t ml = std::min<size_t>(std::strlen(magic), 8);
  if (len < 24) return Corrupt("file shorter than its header");
  if (std::memcmp(p, magic, ml) != 0) return Corrupt("bad file magic");
  if (Get<uint32_t>(p + 8) != 1) return Corrupt("unsupported file version");
  if (Get<uint64_t>(p + 16) != len - 24) return Corrupt("file length mismatch");
  if (vdbg::Crc32c(p + 24, len - 24) != Get<uint32_t>(p + 12)) return Corrupt("file checksum mismatch");
  *payload_offset = 24;
  *payload_len = len - 24;
  return VDBG_OK;
}

int vdbg_deletes_decode(const void* file, size_t len, size_t rows, uint64_t* deleted_words,
                        uint64_t* count) {
  if (deleted_words == nullptr && rows > 0)
    return vdbg::SetError(VDBG_INVALID_ARGUMENT, "null argument");
  size_t off = 0, plen = 0;
  const int rc = vdbg_blob_decode(file, len, "VDBDEL01", &off, &plen);
  if (rc != VDBG_OK) return rc;
  const uint8_t* p = static_cast<const uint8_t*>(file) + off;
  const size_t nwords = (rows + 63) / 64;
  if (nwords > 0) std::memset(deleted_words, 0, nwords * sizeof(uint64_t));

  // ---- cookie and container count
  constexpr uint32_t kNoRunCookie = 12346, kRunCookie = 12347;
  constexpr size_t kNoOffsetThreshold = 4, kArrayMax = 4096;
  auto bad = [] { return Corrupt("bad delete set: malformed roaring bitmap"); };
  size_t pos = 0;
  auto need = [&](size_t b) { return plen - pos >= b; };
  if (!need(4)) return bad();
  const uint32_t cookie = Get<uint32_t>(p);
  pos = 4;
  size_t size = 0;
  const uint8_t* runflags = nullptr;
  if ((cookie & 0xffffu) == kRunCookie) {
    size = (cookie >> 16) + 1;
    if (!need((size + 7) / 8)) return bad();
    runflags = p + pos;
    pos += (size + 7) / 8;
  } else if (cookie == kNoRunCookie) {
    if (!need(4)) return bad();
    size = Get<uint32_t>(p + pos);
    pos += 4;
  } else {
    return bad();
  }
  if (size > 65536) return bad();

  // ---- descriptive header, then the offset header (skipped: containers are read in order)
  if (!need(size * 4)) return bad();
  const uint8_t* desc = p + pos;
  pos += size * 4;
  if (runflags == nullptr || size >= kNoOffsetThreshold) {
    if (!need(size * 4)) return bad();
    pos += size * 4;
  }

  uint64_t total = 0;
  auto mark = [&](uint32_t v) -> bool {
    if (v >= rows) return false;
    uint64_t& w = deleted_words[v >> 6];
    const uint64_t bit = uint64_t(1) << (v & 63);
    total += (w & bit) ? 0 : 1;
    w |= bit;
    return true;
  };
  auto range = [] { return Corrupt("delete set out of range"); };
  for (size_t i = 0; i < size; ++i) {
    const uint32_t key = Get<uint16_t>(desc + 4 * i);
    const size_t card = size_t(Get<uint16_t>(desc + 4 * i + 2)) + 1;
    const uint32_t hi = key << 16;
    if (runflags != nullptr && ((runflags[i >> 3] >> (i & 7)) & 1u)) {
      if (!need(2)) return bad();
      const size_t nruns = Get<uint16_t>(p + pos);
      pos += 2;
      if (!need(nruns * 4)) return bad();
      for (size_t r = 0; r < nruns; ++r) {
        const uint32_t start = Get<uint16_t>(p + pos + 4 * r);
        const uint32_t length = Get<uint16_t>(p + pos + 4 * r + 2);
        if (start + length > 0xffffu) return bad();
        for (uint32_t v = start; v <= start + length; ++v)
          if (!mark(hi | v)) return range();
      }
      pos += nruns * 4;
    } else if (card <= kArrayMax) {
      if (!need(card * 2)) return bad();
      for (size_t j = 0; j < card; ++j)
        if (!mark(hi | Get<uint16_t>(p + pos + 2 * j))) return range();
      pos += card * 2;
    } else {
      if (!need(8192)) return bad();
      for (uint32_t w = 0; w < 1024; ++w) {
        uint64_t bits = Get<uint64_t>(p + pos + 8 * size_t(w));
        while (bits != 0) {
          if (!mark(hi | (w << 6) | uint32_t(__builtin_ctzll(bits)))) return range();
          bits &= bits - 1;
        }
      }
      pos += 8192;
    }
  }
  if (count != nullptr) *count = total;
  return VDBG_OK;
}

}  // extern "C"
