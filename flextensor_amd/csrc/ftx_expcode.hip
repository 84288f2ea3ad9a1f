// Exponent-coded blocks: a lossless encoding of streamed bf16 weight blocks
// that carries about three quarters of the raw bytes over the host link, and
// the zero-copy kernel that decodes one straight from mapped host memory into
// its ring slot.
//
// bf16 weights drawn from one distribution use few exponents: the 7B-shape
// layers (N(0, 0.02)) have about 2.5 bits of exponent entropy and 15
// exponents cover all but 0.02% of their words. A block of N raw bytes is read
// as W = N / 2 little-endian 16-bit words (sign bit 15, exponent 14..7,
// mantissa 6..0) in groups of 1024 words; an odd last byte is kept verbatim:
//
//   header (64 bytes, zero padded to 256): "FTXE", u32 version 1, u64 N, u64 W,
//       u64 G (groups), u64 E (escapes), table[16], u8 tail byte, 7 zero bytes
//   plane A at 256:           G*1024 bytes, sign << 7 | mantissa of each word
//   plane B at 256 + 1024 G:  G*512 bytes, a 4-bit code per word (low nibble
//                             first): code c < 15 is exponent table[c], 15 an
//                             escape
//   S at 256 + 1536 G:        G + 1 u32, escapes before each group
//   X at S + align16(4 (G+1)): E u32, (word % 1024) << 8 | exponent, one per
//                             escaped word in word order
//
// The table holds the 15 most frequent exponents, most frequent first, ties to
// the smaller exponent. The encoded size is 256 + 1536 G + align16(4 (G+1)) +
// 4 E bytes. Lane l of a wave decodes words [8l, 8l + 8) and [512 + 8l,
// 512 + 8l + 8) of a group: it reads 8 bytes of plane A and 4 of plane B for
// each run (coalesced across the wave), rebuilds the 16 words in registers and
// writes each run with one 16-byte non-temporal store, so every store
// instruction of the wave covers one contiguous KiB and HBM is written once
// per byte. A group's escapes, when it has any, are patched from X. Each lane
// holds eight groups' loads in flight.
#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "ftx_internal.h"

namespace ftx {

namespace {

struct ExpHeader {
  char magic[4];
  uint32_t version;
  uint64_t n;
  uint64_t n_words;
  uint64_t groups;
  uint64_t escapes;
  uint8_t table[16];
  uint8_t tail;
  uint8_t pad[7];
};
static_assert(sizeof(ExpHeader) == 64, "header layout");

constexpr uint32_t kExpVersion = 1;
constexpr uint32_t kExpEscape = 15;

void sections(uint64_t groups, uint64_t escapes, ExpcodeInfo *p) {
  p->off_b = kExpcodeHeaderBytes + kExpcodeGroupWords * groups;
  p->off_s = p->off_b + kExpcodeGroupWords / 2 * groups;
  p->off_x = p->off_s + (4 * (groups + 1) + 15) / 16 * 16;
  p->total = p->off_x + 4 * escapes;
}

inline uint32_t word_at(const uint8_t *raw, uint64_t w) {
  return static_cast<uint32_t>(raw[2 * w]) | (static_cast<uint32_t>(raw[2 * w + 1]) << 8);
}

// Runs f(begin, end) over [0, n) on up to `threads` threads (the caller is one).
template <class F>
void parallel_for(uint64_t n, int threads, F f) {
  if (threads <= 1 || n < 2) {
    f(0, n);
    return;
  }
  const uint64_t t = std::min<uint64_t>(static_cast<uint64_t>(threads), n);
  const uint64_t chunk = (n + t - 1) / t;
  std::vector<std::thread> pool;
  for (uint64_t i = 1; i < t; ++i) {
    const uint64_t b = i * chunk, e = std::min(n, b + chunk);
    if (b < e) pool.emplace_back([=] { f(b, e); });
  }
  f(0, std::min(n, chunk));
  for (auto &th : pool) th.join();
}

int encode_threads(uint64_t n_words) {
  if (n_words < (uint64_t(1) << 20)) return 1;
  const unsigned hw = std::thread::hardware_concurrency();
  return static_cast<int>(std::clamp<unsigned>(hw / 2, 1u, 16u));
}

// Exponent histogram, table and sizes of a raw block.
struct ExpPlan {
  ExpcodeInfo info;
  uint8_t code_of[256];
};

// Exponent histogram of the first n_words words of raw (threaded above a million words), and the exponents
// that occur, most frequent first, ties to the smaller exponent.
void exponent_ranks(const uint8_t *raw, uint64_t n_words, uint64_t hist[256], std::vector<int> *ranked) {
  const int threads = encode_threads(n_words);
  std::vector<uint64_t> hists(static_cast<size_t>(std::max(threads, 1)) * 256, 0);
  const uint64_t chunk = (n_words + threads - 1) / std::max(threads, 1);
  parallel_for(n_words, threads, [&](uint64_t b, uint64_t e) {
    uint64_t *h = hists.data() + (chunk ? b / chunk : 0) * 256;
    for (uint64_t w = b; w < e; ++w) ++h[(word_at(raw, w) >> 7) & 0xff];
  });
  for (int x = 0; x < 256; ++x) hist[x] = 0;
  for (int t = 0; t < threads; ++t)
    for (int x = 0; x < 256; ++x) hist[x] += hists[static_cast<size_t>(t) * 256 + x];
  ranked->clear();
  for (int x = 0; x < 256; ++x)
    if (hist[x]) ranked->push_back(x);
  std::stable_sort(ranked->begin(), ranked->end(), [&](int a, int b) { return hist[a] > hist[b]; });
}

int plan(const uint8_t *raw, uint64_t n, ExpPlan *p) {
  ExpcodeInfo &info = p->info;
  info = ExpcodeInfo{};
  info.n = n;
  info.n_words = n / 2;
  info.groups = (info.n_words + kExpcodeGroupWords - 1) / kExpcodeGroupWords;
  if (info.groups >= (uint64_t(1) << 32)) return fail(FTX_ERR_INVALID, "block too large to encode");
  uint64_t hist[256];
  std::vector<int> ranked;
  exponent_ranks(raw, info.n_words, hist, &ranked);
  std::memset(p->code_of, kExpEscape, sizeof(p->code_of));
  uint64_t covered = 0;
  for (size_t c = 0; c < ranked.size() && c < kExpEscape; ++c) {
    info.table[c] = static_cast<uint8_t>(ranked[c]);
    p->code_of[ranked[c]] = static_cast<uint8_t>(c);
    covered += hist[ranked[c]];
  }
  info.escapes = info.n_words - covered;
  if (info.escapes >= (uint64_t(1) << 32)) return fail(FTX_ERR_INVALID, "block has too many escaped words to encode");
  info.tail = n % 2 ? raw[n - 1] : 0;
  sections(info.groups, info.escapes, &info);
  return FTX_OK;
}

}  // namespace

int expcode_encode(const void *raw_v, size_t nbytes, void *out_v, size_t out_capacity, size_t *out_bytes) {
  const auto *raw = static_cast<const uint8_t *>(raw_v);
  ExpPlan p;
  int rc = plan(raw, nbytes, &p);
  if (rc != FTX_OK) return rc;
  const ExpcodeInfo &info = p.info;
  *out_bytes = static_cast<size_t>(info.total);
  if (out_v == nullptr) return FTX_OK;
  if (out_capacity < info.total)
    return fail(FTX_ERR_INVALID, "output buffer of " + std::to_string(out_capacity) + " bytes is smaller than the " +
                                     std::to_string(info.total) + " the encoded block needs");
  auto *out = static_cast<uint8_t *>(out_v);
  std::memset(out, 0, kExpcodeHeaderBytes);
  ExpHeader h{};
  std::memcpy(h.magic, "FTXE", 4);
  h.version = kExpVersion;
  h.n = info.n;
  h.n_words = info.n_words;
  h.groups = info.groups;
  h.escapes = info.escapes;
  std::memcpy(h.table, info.table, 16);
  h.tail = info.tail;
  std::memcpy(out, &h, sizeof(h));
  const uint64_t G = info.groups, W = info.n_words;
  std::vector<uint32_t> counts(static_cast<size_t>(G), 0);
  const int threads = encode_threads(W);
  uint8_t *A = out + kExpcodeHeaderBytes, *B = out + info.off_b;
  parallel_for(G, threads, [&](uint64_t gb, uint64_t ge) {
    for (uint64_t g = gb; g < ge; ++g) {
      const uint64_t w0 = g * kExpcodeGroupWords;
      const uint64_t wn = std::min<uint64_t>(kExpcodeGroupWords, W - w0);
      uint32_t cnt = 0;
      const uint64_t whole = wn / 8 * 8;  // words handled eight at a time: one 16-byte load, 8 + 4 bytes out
      for (uint64_t j = 0; j < whole; j += 8) {
        uint16_t w[8];
        std::memcpy(w, raw + 2 * (w0 + j), 16);
        uint64_t a8 = 0;
        uint32_t c8 = 0;
        for (int k = 0; k < 8; ++k) {
          const uint32_t word = w[k];
          const uint32_t c = p.code_of[(word >> 7) & 0xff];
          a8 |= static_cast<uint64_t>(((word >> 8) & 0x80) | (word & 0x7f)) << (8 * k);
          c8 |= c << (4 * k);
          cnt += c == kExpEscape;
        }
        std::memcpy(A + w0 + j, &a8, 8);
        std::memcpy(B + (w0 + j) / 2, &c8, 4);
      }
      for (uint64_t j = whole; j < kExpcodeGroupWords; j += 2) {  // the last words, and zeros past them
        uint32_t c[2] = {0, 0};
        for (int k = 0; k < 2; ++k) {
          uint8_t a = 0;
          if (j + k < wn) {
            const uint32_t word = word_at(raw, w0 + j + k);
            a = static_cast<uint8_t>(((word >> 8) & 0x80) | (word & 0x7f));
            c[k] = p.code_of[(word >> 7) & 0xff];
            cnt += c[k] == kExpEscape;
          }
          A[w0 + j + k] = a;
        }
        B[(w0 + j) / 2] = static_cast<uint8_t>(c[0] | (c[1] << 4));
      }
      counts[static_cast<size_t>(g)] = cnt;
    }
  });
  std::vector<uint32_t> S(static_cast<size_t>(G) + 1, 0);
  for (uint64_t g = 0; g < G; ++g) S[static_cast<size_t>(g) + 1] = S[static_cast<size_t>(g)] + counts[static_cast<size_t>(g)];
  if (S[static_cast<size_t>(G)] != info.escapes) return fail(FTX_ERR_INVALID, "escape count mismatch while encoding");
  std::memset(out + info.off_s, 0, static_cast<size_t>(info.off_x - info.off_s));
  std::memcpy(out + info.off_s, S.data(), S.size() * sizeof(uint32_t));
  uint8_t *X = out + info.off_x;
  parallel_for(G, threads, [&](uint64_t gb, uint64_t ge) {
    for (uint64_t g = gb; g < ge; ++g) {
      if (!counts[static_cast<size_t>(g)]) continue;
      const uint64_t w0 = g * kExpcodeGroupWords;
      const uint64_t wn = std::min<uint64_t>(kExpcodeGroupWords, W - w0);
      uint64_t k = S[static_cast<size_t>(g)];
      for (uint64_t j = 0; j < wn; ++j) {
        const uint32_t e = (word_at(raw, w0 + j) >> 7) & 0xff;
        if (p.code_of[e] != kExpEscape) continue;
        const uint32_t x = static_cast<uint32_t>(j << 8) | e;
        std::memcpy(X + 4 * k, &x, 4);
        ++k;
      }
    }
  });
  return FTX_OK;
}

namespace {

struct DenseHeader {
  char magic[4];
  uint32_t version;
  uint64_t n;
  uint64_t n_words;
  uint64_t groups;
  uint64_t e1;  // primary escapes
  uint64_t e2;  // secondary escapes
  uint8_t t1[8];
  uint8_t t2[16];
  uint8_t tail;
  uint8_t pad[7];
};
static_assert(sizeof(DenseHeader) == 80, "dense header layout");

constexpr uint32_t kDenseVersion = 2;
constexpr uint32_t kPrimaryEscape = 7;
constexpr uint32_t kSecondaryEscape = 15;

}  // namespace

DenseLayout dense_layout(uint64_t n, uint64_t e1, uint64_t e2) {
  DenseLayout d{};
  d.n = n;
  d.n_words = n / 2;
  d.groups = (d.n_words + kExpcodeGroupWords - 1) / kExpcodeGroupWords;
  d.e1 = e1;
  d.e2 = e2;
  const uint64_t s = (4 * (d.groups + 1) + 15) / 16 * 16;
  d.off_p = kExpcodeHeaderBytes + kExpcodeGroupWords * d.groups;
  d.off_s1 = d.off_p + kDensePlaneBytes * d.groups;
  d.off_s2 = d.off_s1 + s;
  d.off_y = d.off_s2 + s;
  d.off_x = d.off_y + ((e1 + 1) / 2 + 15) / 16 * 16;
  d.total = d.off_x + 4 * e2;
  return d;
}

int expcode_encode_dense(const void *raw_v, size_t nbytes, void *out_v, size_t out_capacity, size_t *out_bytes) {
  const auto *raw = static_cast<const uint8_t *>(raw_v);
  const uint64_t W = nbytes / 2;
  const uint64_t G = (W + kExpcodeGroupWords - 1) / kExpcodeGroupWords;
  if (G >= (uint64_t(1) << 32)) return fail(FTX_ERR_INVALID, "block too large to encode");
  uint64_t hist[256];
  std::vector<int> ranked;
  exponent_ranks(raw, W, hist, &ranked);
  uint8_t code1[256], code2[256];
  std::memset(code1, kPrimaryEscape, sizeof(code1));
  std::memset(code2, kSecondaryEscape, sizeof(code2));
  DenseHeader h{};
  std::memcpy(h.magic, "FTXE", 4);
  h.version = kDenseVersion;
  uint64_t covered1 = 0, covered2 = 0;
  for (size_t c = 0; c < ranked.size() && c < kPrimaryEscape + kSecondaryEscape; ++c) {
    const int e = ranked[c];
    if (c < kPrimaryEscape) {
      h.t1[c] = static_cast<uint8_t>(e);
      code1[e] = static_cast<uint8_t>(c);
      covered1 += hist[e];
    } else {
      h.t2[c - kPrimaryEscape] = static_cast<uint8_t>(e);
      code2[e] = static_cast<uint8_t>(c - kPrimaryEscape);
      covered2 += hist[e];
    }
  }
  const uint64_t e1 = W - covered1, e2 = e1 - covered2;
  if (e1 >= (uint64_t(1) << 32)) return fail(FTX_ERR_INVALID, "block has too many escaped words to encode");
  const DenseLayout d = dense_layout(nbytes, e1, e2);
  *out_bytes = static_cast<size_t>(d.total);
  if (out_v == nullptr) return FTX_OK;
  if (out_capacity < d.total)
    return fail(FTX_ERR_INVALID, "output buffer of " + std::to_string(out_capacity) + " bytes is smaller than the " +
                                     std::to_string(d.total) + " the encoded block needs");
  auto *out = static_cast<uint8_t *>(out_v);
  std::memset(out, 0, kExpcodeHeaderBytes);
  h.n = nbytes;
  h.n_words = W;
  h.groups = G;
  h.e1 = e1;
  h.e2 = e2;
  h.tail = nbytes % 2 ? raw[nbytes - 1] : 0;
  std::memcpy(out, &h, sizeof(h));
  std::vector<uint32_t> count1(static_cast<size_t>(G), 0), count2(static_cast<size_t>(G), 0);
  const int threads = encode_threads(W);
  uint8_t *A = out + kExpcodeHeaderBytes, *P = out + d.off_p;
  // Plane A and the code bit planes, eight words (one byte of each plane) at a time.
  parallel_for(G, threads, [&](uint64_t gb, uint64_t ge) {
    for (uint64_t g = gb; g < ge; ++g) {
      const uint64_t w0 = g * kExpcodeGroupWords;
      const uint64_t wn = std::min<uint64_t>(kExpcodeGroupWords, W - w0);
      uint32_t c1 = 0, c2 = 0;
      uint8_t *planes = P + g * kDensePlaneBytes;
      for (uint64_t i = 0; i < kExpcodeGroupWords / 8; ++i) {
        uint32_t b0 = 0, b1 = 0, b2 = 0;
        for (uint64_t k = 0; k < 8; ++k) {
          const uint64_t j = 8 * i + k;
          uint8_t a = 0;
          if (j < wn) {
            const uint32_t word = word_at(raw, w0 + j);
            const uint32_t e = (word >> 7) & 0xff;
            const uint32_t c = code1[e];
            a = static_cast<uint8_t>(((word >> 8) & 0x80) | (word & 0x7f));
            b0 |= (c & 1) << k;
            b1 |= ((c >> 1) & 1) << k;
            b2 |= ((c >> 2) & 1) << k;
            if (c == kPrimaryEscape) {
              ++c1;
              c2 += code2[e] == kSecondaryEscape;
            }
          }
          A[w0 + j] = a;
        }
        const uint64_t at = 2 * (i % 64) + i / 64;  // words 512 h + 8 l .. : byte 2 l + h of each plane
        planes[at] = static_cast<uint8_t>(b0);
        planes[128 + at] = static_cast<uint8_t>(b1);
        planes[256 + at] = static_cast<uint8_t>(b2);
      }
      count1[static_cast<size_t>(g)] = c1;
      count2[static_cast<size_t>(g)] = c2;
    }
  });
  std::vector<uint32_t> S1(static_cast<size_t>(G) + 1, 0), S2(static_cast<size_t>(G) + 1, 0);
  for (uint64_t g = 0; g < G; ++g) {
    S1[static_cast<size_t>(g) + 1] = S1[static_cast<size_t>(g)] + count1[static_cast<size_t>(g)];
    S2[static_cast<size_t>(g) + 1] = S2[static_cast<size_t>(g)] + count2[static_cast<size_t>(g)];
  }
  if (S1[static_cast<size_t>(G)] != e1 || S2[static_cast<size_t>(G)] != e2)
    return fail(FTX_ERR_INVALID, "escape count mismatch while encoding");
  std::memset(out + d.off_s1, 0, static_cast<size_t>(d.off_x - d.off_s1));
  std::memcpy(out + d.off_s1, S1.data(), S1.size() * sizeof(uint32_t));
  std::memcpy(out + d.off_s2, S2.data(), S2.size() * sizeof(uint32_t));
  uint8_t *Y = out + d.off_y, *X = out + d.off_x;
  // The secondary codes and the list. A byte of Y holds two nibbles; the bytes at the ends of a thread's
  // range of nibbles may hold a neighbouring range's nibble too, and take their nibble by an atomic or.
  parallel_for(G, threads, [&](uint64_t gb, uint64_t ge) {
    const uint64_t lo = S1[static_cast<size_t>(gb)], hi = S1[static_cast<size_t>(ge)];
    if (lo == hi) return;
    const uint64_t edge_lo = lo / 2, edge_hi = (hi - 1) / 2;
    for (uint64_t g = gb; g < ge; ++g) {
      if (!count1[static_cast<size_t>(g)]) continue;
      const uint64_t w0 = g * kExpcodeGroupWords;
      const uint64_t wn = std::min<uint64_t>(kExpcodeGroupWords, W - w0);
      uint64_t r = S1[static_cast<size_t>(g)], x = S2[static_cast<size_t>(g)];
      for (uint64_t j = 0; j < wn; ++j) {
        const uint32_t e = (word_at(raw, w0 + j) >> 7) & 0xff;
        if (code1[e] != kPrimaryEscape) continue;
        const uint32_t c = code2[e];
        const uint8_t bits = static_cast<uint8_t>(c << (4 * (r & 1)));
        if (r / 2 == edge_lo || r / 2 == edge_hi)
          __atomic_fetch_or(Y + r / 2, bits, __ATOMIC_RELAXED);
        else
          Y[r / 2] |= bits;
        ++r;
        if (c == kSecondaryEscape) {
          const uint32_t v = static_cast<uint32_t>(j << 8) | e;
          std::memcpy(X + 4 * x, &v, 4);
          ++x;
        }
      }
    }
  });
  return FTX_OK;
}

int expcode_parse_dense(const void *src, size_t src_bytes, DenseLayout *layout) {
  if (src_bytes < kExpcodeHeaderBytes) return fail(FTX_ERR_INVALID, "encoded block shorter than its header");
  DenseHeader h;
  std::memcpy(&h, src, sizeof(h));
  if (std::memcmp(h.magic, "FTXE", 4) != 0 || h.version != kDenseVersion)
    return fail(FTX_ERR_INVALID, "not a dense exponent-coded block (magic or version)");
  if (h.n_words != h.n / 2 || h.groups != (h.n_words + kExpcodeGroupWords - 1) / kExpcodeGroupWords ||
      h.groups >= (uint64_t(1) << 32) || h.e1 > h.n_words || h.e1 >= (uint64_t(1) << 32) || h.e2 > h.e1)
    return fail(FTX_ERR_INVALID, "inconsistent dense exponent-coded block header");
  *layout = dense_layout(h.n, h.e1, h.e2);
  if (layout->total > src_bytes) return fail(FTX_ERR_INVALID, "encoded block is truncated");
  return FTX_OK;
}

int expcode_parse(const void *src, size_t src_bytes, ExpcodeInfo *info) {
  if (src_bytes < kExpcodeHeaderBytes) return fail(FTX_ERR_INVALID, "encoded block shorter than its header");
  ExpHeader h;
  std::memcpy(&h, src, sizeof(h));
  if (std::memcmp(h.magic, "FTXE", 4) != 0 || h.version != kExpVersion)
    return fail(FTX_ERR_INVALID, "not an exponent-coded block (magic or version)");
  if (h.n_words != h.n / 2 || h.groups != (h.n_words + kExpcodeGroupWords - 1) / kExpcodeGroupWords ||
      h.groups >= (uint64_t(1) << 32) || h.escapes > h.n_words || h.escapes >= (uint64_t(1) << 32))
    return fail(FTX_ERR_INVALID, "inconsistent exponent-coded block header");
  *info = ExpcodeInfo{};
  info->n = h.n;
  info->n_words = h.n_words;
  info->groups = h.groups;
  info->escapes = h.escapes;
  std::memcpy(info->table, h.table, 16);
  info->tail = h.tail;
  sections(h.groups, h.escapes, info);
  if (info->total > src_bytes) return fail(FTX_ERR_INVALID, "encoded block is truncated");
  return FTX_OK;
}

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kExpThreads = 512;  // 8 waves: 16 workgroups reach the link peak (4 waves: 0.8% slower, 16 waves: no faster)
constexpr int kExpWaves = kExpThreads / 64;
constexpr int kExpInFlight = 8;  // groups whose loads each lane keeps in flight

__device__ __forceinline__ uint32_t decode_word(uint32_t a, uint32_t code, uint64_t t01, uint64_t t23) {
  const uint64_t t = code < 8 ? t01 : t23;
  const uint32_t e = static_cast<uint32_t>(t >> ((code & 7) * 8)) & 0xff;
  return ((a & 0x80) << 8) | (e << 7) | (a & 0x7f);
}

// Wave w decodes groups w*8 .. w*8+7, then steps by 8 x (waves in the grid).
// Loads of groups past the last read the last group (in bounds) and are
// discarded. The sections follow from the raw size n; the
// escape count, table and tail byte are read from the block's header when the
// kernel runs, so a graph that captured the launch decodes the block's
// current contents after it is re-encoded in place. A header of another raw
// size writes nothing, and escape reads stay inside `capacity` bytes.
__global__ __launch_bounds__(kExpThreads) void expcode_decode_kernel(uint8_t *__restrict__ dst,
                                                                     const uint8_t *__restrict__ src,
                                                                     uint64_t capacity, uint64_t n) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = static_cast<uint64_t>(blockIdx.x) * kExpWaves + threadIdx.x / 64;
  const uint64_t waves = static_cast<uint64_t>(gridDim.x) * kExpWaves;
  const uint64_t n_words = n / 2;
  const uint64_t groups = (n_words + kExpcodeGroupWords - 1) / kExpcodeGroupWords;
  const uint64_t off_b = kExpcodeHeaderBytes + kExpcodeGroupWords * groups;
  const uint64_t off_s = off_b + kExpcodeGroupWords / 2 * groups;
  const uint64_t off_x = off_s + (4 * (groups + 1) + 15) / 16 * 16;
  if (*reinterpret_cast<const uint64_t *>(src + 8) != n) return;
  uint64_t escapes = *reinterpret_cast<const uint64_t *>(src + 32);
  escapes = off_x <= capacity ? min(escapes, (capacity - off_x) / 4) : 0;
  const uint64_t t01 = *reinterpret_cast<const uint64_t *>(src + 40);
  const uint64_t t23 = *reinterpret_cast<const uint64_t *>(src + 48);
  if ((n & 1) && blockIdx.x == 0 && threadIdx.x == 0) dst[n - 1] = src[56];
  const uint8_t *A = src + kExpcodeHeaderBytes;
  const uint8_t *B = src + off_b;
  const uint32_t *S = reinterpret_cast<const uint32_t *>(src + off_s);
  const uint32_t *X = reinterpret_cast<const uint32_t *>(src + off_x);
  // Lane l decodes two runs of 8 words, [8l, 8l + 8) and [512 + 8l, 512 + 8l + 8) of the group, so that each
  // 16-byte store instruction of the wave writes one contiguous KiB.
  for (uint64_t g0 = wave * kExpInFlight; g0 < groups; g0 += waves * kExpInFlight) {
    u32x2 a[kExpInFlight][2];
    uint32_t b[kExpInFlight][2];
#pragma unroll
    for (int i = 0; i < kExpInFlight; ++i) {
      const uint64_t g = min(g0 + i, groups - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        a[i][h] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x2 *>(A + g * kExpcodeGroupWords + 512 * h) + lane);
        b[i][h] = __builtin_nontemporal_load(
            reinterpret_cast<const uint32_t *>(B + g * (kExpcodeGroupWords / 2) + 256 * h) + lane);
      }
    }
    // S[g0 .. g0 + 8], one entry per lane (lanes past them repeat the last), clamped to S[G]
    const uint32_t sv = S[min(g0 + min(lane, kExpInFlight), groups)];
#pragma unroll
    for (int i = 0; i < kExpInFlight; ++i) {
      const uint64_t g = g0 + i;
      if (g >= groups) break;
      uint32_t word[16];  // run h, word j at 8h + j
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          word[8 * h + j] = decode_word((a[i][h][j >> 2] >> (8 * (j & 3))) & 0xff, (b[i][h] >> (4 * j)) & 0xf, t01, t23);
      const uint32_t s0 = __shfl(sv, i, 64);
      const uint32_t s1 = min(static_cast<uint64_t>(__shfl(sv, i + 1, 64)), escapes);
      for (uint32_t k = s0; k < s1; ++k) {  // wave-uniform; escapes are rare
        const uint32_t x = X[k];
        const uint32_t pos = x >> 8;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (pos == static_cast<uint32_t>(512 * h + 8 * lane + j))
              word[8 * h + j] = (word[8 * h + j] & 0x807fu) | ((x & 0xffu) << 7);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint64_t w0 = g * kExpcodeGroupWords + 512 * h + 8 * static_cast<uint64_t>(lane);
        uint8_t *out = dst + 2 * w0;
        if (w0 + 8 <= n_words) {
          u32x4 v;
#pragma unroll
          for (int k = 0; k < 4; ++k) v[k] = word[8 * h + 2 * k] | (word[8 * h + 2 * k + 1] << 16);
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(out));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (w0 + j < n_words) reinterpret_cast<uint16_t *>(out)[j] = static_cast<uint16_t>(word[8 * h + j]);
        }
      }
    }
  }
}

constexpr int kDenseInFlight = 4;  // groups whose loads each lane keeps in flight (the source is HBM)

// Dense blocks (version 2) from device memory. The same group walk and store mapping as
// expcode_decode_kernel: lane l decodes runs h = 0, 1 of words [512h + 8l, 512h + 8l + 8) of each group,
// four words to a register with byte permutes (a 7B layer: 172 us, against 209 word by word).
// A lane's primary codes are one 16-bit value per bit plane (byte h for run h); the escape mask of a run is
// the AND of its three bytes. A primary escape's secondary code is the nibble at its rank in word order:
// S1 of its group, plus the escapes of earlier runs and lanes (one inclusive scan of the packed per-lane
// counts across the wave), plus those before it in its own run. Ranks and list reads are clamped to
// `capacity`; a header of another raw size writes nothing.
__global__ __launch_bounds__(kExpThreads) void expcode_dense_decode_kernel(uint8_t *__restrict__ dst,
                                                                           const uint8_t *__restrict__ src,
                                                                           uint64_t capacity, uint64_t n) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = static_cast<uint64_t>(blockIdx.x) * kExpWaves + threadIdx.x / 64;
  const uint64_t waves = static_cast<uint64_t>(gridDim.x) * kExpWaves;
  const uint64_t n_words = n / 2;
  const uint64_t groups = (n_words + kExpcodeGroupWords - 1) / kExpcodeGroupWords;
  const uint64_t sect = (4 * (groups + 1) + 15) / 16 * 16;
  const uint64_t off_p = kExpcodeHeaderBytes + kExpcodeGroupWords * groups;
  const uint64_t off_s1 = off_p + kDensePlaneBytes * groups;
  const uint64_t off_s2 = off_s1 + sect;
  const uint64_t off_y = off_s2 + sect;
  if (off_y > capacity || *reinterpret_cast<const uint64_t *>(src + 8) != n) return;
  const uint64_t e1 = *reinterpret_cast<const uint64_t *>(src + 32);
  const uint64_t off_x = off_y + ((min(e1, capacity) + 1) / 2 + 15) / 16 * 16;
  uint64_t e2 = *reinterpret_cast<const uint64_t *>(src + 40);
  e2 = off_x <= capacity ? min(e2, (capacity - off_x) / 4) : 0;
  const uint64_t y_bytes = capacity - off_y;
  const uint32_t t1_lo = *reinterpret_cast<const uint32_t *>(src + 48);
  const uint32_t t1_hi = *reinterpret_cast<const uint32_t *>(src + 52);
  const uint32_t t2a_lo = *reinterpret_cast<const uint32_t *>(src + 56);
  const uint32_t t2a_hi = *reinterpret_cast<const uint32_t *>(src + 60);
  const uint32_t t2b_lo = *reinterpret_cast<const uint32_t *>(src + 64);
  const uint32_t t2b_hi = *reinterpret_cast<const uint32_t *>(src + 68);
  if ((n & 1) && blockIdx.x == 0 && threadIdx.x == 0) dst[n - 1] = src[72];
  const uint8_t *A = src + kExpcodeHeaderBytes;
  const uint8_t *P = src + off_p;
  const uint32_t *S1 = reinterpret_cast<const uint32_t *>(src + off_s1);
  const uint32_t *S2 = reinterpret_cast<const uint32_t *>(src + off_s2);
  const uint8_t *Y = src + off_y;
  const uint32_t *X = reinterpret_cast<const uint32_t *>(src + off_x);
  for (uint64_t g0 = wave * kDenseInFlight; g0 < groups; g0 += waves * kDenseInFlight) {
    u32x2 a[kDenseInFlight][2];
    uint32_t pw[kDenseInFlight][3];  // plane k: run 0's code bits in the low byte, run 1's in the next
#pragma unroll
    for (int i = 0; i < kDenseInFlight; ++i) {
      const uint64_t g = min(g0 + i, groups - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        a[i][h] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x2 *>(A + g * kExpcodeGroupWords + 512 * h) + lane);
#pragma unroll
      for (int k = 0; k < 3; ++k)
        pw[i][k] = reinterpret_cast<const uint16_t *>(P + g * kDensePlaneBytes + 128 * k)[lane];
    }
    // S1 and S2 at g0 .. g0 + kDenseInFlight, one entry per lane, clamped to the last
    const uint64_t si = min(g0 + min(lane, kDenseInFlight), groups);
    const uint32_t s1v = S1[si], s2v = S2[si];
#pragma unroll
    for (int i = 0; i < kDenseInFlight; ++i) {
      const uint64_t g = g0 + i;
      if (g >= groups) break;
      // Exponents four words to a register, one byte each: the three code bits of words 4q .. 4q + 3 spread
      // into bytes (a multiply by 0x00204081 moves bit j to bit 8j without carries), then one byte permute
      // picks each word's exponent from T1. Escapes (code 7) pick T1[7] = 0 and are set below.
      uint32_t ex[2][2];  // run h, quad q
      uint32_t mask[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        mask[h] = (pw[i][0] & pw[i][1] & pw[i][2]) >> (8 * h) & 0xff;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          uint32_t codes = 0;
#pragma unroll
          for (int k = 0; k < 3; ++k) codes |= ((((pw[i][k] >> (8 * h + 4 * q)) & 0xf) * 0x00204081u) & 0x01010101u) << k;
          ex[h][q] = __builtin_amdgcn_perm(t1_hi, t1_lo, codes);
        }
      }
      const uint32_t s1a = __shfl(s1v, i, 64), s1b = __shfl(s1v, i + 1, 64);
      if (s1b > s1a) {  // wave-uniform: the group has primary escapes
        const uint32_t cnt = __popc(mask[0]) | (__popc(mask[1]) << 16);
        uint32_t incl = cnt;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const uint32_t y = __shfl_up(incl, d, 64);
          if (lane >= d) incl += y;
        }
        const uint32_t excl = incl - cnt;
        const uint32_t run0 = __shfl(incl, 63, 64) & 0xffff;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint64_t r = static_cast<uint64_t>(s1a) + (h ? run0 + (excl >> 16) : (excl & 0xffff));
          uint32_t m = mask[h];
          while (m) {
            const int j = __builtin_ctz(m);
            m &= m - 1;
            const uint32_t yb = (r >> 1) < y_bytes ? Y[r >> 1] : 0u;
            const uint32_t c2 = (yb >> (4 * (r & 1))) & 0xf;
            const uint32_t e = __builtin_amdgcn_perm(c2 < 8 ? t2a_hi : t2b_hi, c2 < 8 ? t2a_lo : t2b_lo, c2 & 7) & 0xff;
            const uint32_t sh = 8 * (j & 3);  // a secondary escape takes T2[15] = 0 here and is patched below
            if (j < 4)
              ex[h][0] = (ex[h][0] & ~(0xffu << sh)) | (e << sh);
            else
              ex[h][1] = (ex[h][1] & ~(0xffu << sh)) | (e << sh);
            ++r;
          }
        }
        const uint32_t s2a = __shfl(s2v, i, 64);
        const uint32_t s2b = min(static_cast<uint64_t>(__shfl(s2v, i + 1, 64)), e2);
        for (uint32_t k = s2a; k < s2b; ++k) {  // wave-uniform; secondary escapes are rarer still
          const uint32_t x = X[k];
          const uint32_t pos = x >> 8;
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (pos == static_cast<uint32_t>(512 * h + 8 * lane + j))
                ex[h][j >> 2] = (ex[h][j >> 2] & ~(0xffu << (8 * (j & 3)))) | ((x & 0xffu) << (8 * (j & 3)));
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint64_t w0 = g * kExpcodeGroupWords + 512 * h + 8 * static_cast<uint64_t>(lane);
        uint8_t *out = dst + 2 * w0;
        // Two words to a register: sign and mantissa bytes and exponent bytes moved into 16-bit lanes by
        // byte permutes (selector 0x0c gives a zero byte), then word = sign << 15 | exponent << 7 | mantissa.
        u32x4 v;
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const uint32_t sel = half ? 0x0c030c02u : 0x0c010c00u;
            const uint32_t av = __builtin_amdgcn_perm(0u, a[i][h][q], sel);
            const uint32_t ev = __builtin_amdgcn_perm(0u, ex[h][q], sel);
            v[2 * q + half] = ((av & 0x00800080u) << 8) | (ev << 7) | (av & 0x007f007fu);
          }
        if (w0 + 8 <= n_words) {
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(out));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (w0 + j < n_words) reinterpret_cast<uint16_t *>(out)[j] = static_cast<uint16_t>(v[j >> 1] >> (16 * (j & 1)));
        }
      }
    }
  }
}

constexpr int kDenseLinkInFlight = 8;  // groups per lane per batch (16 made the compiler spill to scratch)

// Dense blocks (version 2) over the link: the source is mapped host memory, so every read is a PCIe round
// trip and a group's nibble reads cannot wait on its own rank scan one group at a time. Each batch of
// kDenseLinkInFlight groups per lane goes in three phases: the plane, code and prefix-count loads of every
// group; the rank scans, then one 8-byte nibble window per run with escapes, all issued together; then the
// words, built four to a register as in expcode_dense_decode_kernel. A run whose escapes pass its window,
// or a window past the block, reads its nibbles byte by byte. Reads are clamped to `capacity`.
__global__ __launch_bounds__(kExpThreads) void expcode_dense_link_decode_kernel(uint8_t *__restrict__ dst,
                                                                                const uint8_t *__restrict__ src,
                                                                                uint64_t capacity, uint64_t n) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = static_cast<uint64_t>(blockIdx.x) * kExpWaves + threadIdx.x / 64;
  const uint64_t waves = static_cast<uint64_t>(gridDim.x) * kExpWaves;
  const uint64_t n_words = n / 2;
  const uint64_t groups = (n_words + kExpcodeGroupWords - 1) / kExpcodeGroupWords;
  const uint64_t sect = (4 * (groups + 1) + 15) / 16 * 16;
  const uint64_t off_p = kExpcodeHeaderBytes + kExpcodeGroupWords * groups;
  const uint64_t off_s1 = off_p + kDensePlaneBytes * groups;
  const uint64_t off_s2 = off_s1 + sect;
  const uint64_t off_y = off_s2 + sect;
  if (off_y > capacity || *reinterpret_cast<const uint64_t *>(src + 8) != n) return;
  const uint64_t e1 = *reinterpret_cast<const uint64_t *>(src + 32);
  const uint64_t off_x = off_y + ((min(e1, capacity) + 1) / 2 + 15) / 16 * 16;
  uint64_t e2 = *reinterpret_cast<const uint64_t *>(src + 40);
  e2 = off_x <= capacity ? min(e2, (capacity - off_x) / 4) : 0;
  const uint64_t y_bytes = capacity - off_y;
  const uint32_t t1_lo = *reinterpret_cast<const uint32_t *>(src + 48);
  const uint32_t t1_hi = *reinterpret_cast<const uint32_t *>(src + 52);
  const uint32_t t2a_lo = *reinterpret_cast<const uint32_t *>(src + 56);
  const uint32_t t2a_hi = *reinterpret_cast<const uint32_t *>(src + 60);
  const uint32_t t2b_lo = *reinterpret_cast<const uint32_t *>(src + 64);
  const uint32_t t2b_hi = *reinterpret_cast<const uint32_t *>(src + 68);
  if ((n & 1) && blockIdx.x == 0 && threadIdx.x == 0) dst[n - 1] = src[72];
  const uint8_t *A = src + kExpcodeHeaderBytes;
  const uint8_t *P = src + off_p;
  const uint32_t *S1 = reinterpret_cast<const uint32_t *>(src + off_s1);
  const uint32_t *S2 = reinterpret_cast<const uint32_t *>(src + off_s2);
  const uint8_t *Y = src + off_y;
  const uint32_t *X = reinterpret_cast<const uint32_t *>(src + off_x);
  constexpr int F = kDenseLinkInFlight;
  for (uint64_t g0 = wave * F; g0 < groups; g0 += waves * F) {
    // phase 1: planes, codes and prefix counts of F groups
    u32x2 a[F][2];
    uint32_t pw[F][3];
#pragma unroll
    for (int i = 0; i < F; ++i) {
      const uint64_t g = min(g0 + i, groups - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        a[i][h] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x2 *>(A + g * kExpcodeGroupWords + 512 * h) + lane);
#pragma unroll
      for (int k = 0; k < 3; ++k)
        pw[i][k] = reinterpret_cast<const uint16_t *>(P + g * kDensePlaneBytes + 128 * k)[lane];
    }
    const uint64_t si = min(g0 + min(lane, F), groups);  // lanes 0 .. F: S1 and S2 at g0 .. g0 + F
    const uint32_t s1v = S1[si], s2v = S2[si];
    // phase 2: ranks, then every run's nibble window
    uint32_t rank0[F][2];
    uint64_t wbase[F][2];
    u32x2 win[F][2];
#pragma unroll
    for (int i = 0; i < F; ++i) {
      const uint32_t m0 = (pw[i][0] & pw[i][1] & pw[i][2]) & 0xff, m1 = (pw[i][0] & pw[i][1] & pw[i][2]) >> 8 & 0xff;
      const uint32_t s1a = __shfl(s1v, i, 64), s1b = __shfl(s1v, i + 1, 64);
      uint32_t excl = 0, run0 = 0;
      if (g0 + i < groups && s1b > s1a) {  // wave-uniform
        const uint32_t cnt = __popc(m0) | (__popc(m1) << 16);
        uint32_t incl = cnt;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const uint32_t y = __shfl_up(incl, d, 64);
          if (lane >= d) incl += y;
        }
        excl = incl - cnt;
        run0 = __shfl(incl, 63, 64) & 0xffff;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint64_t r = static_cast<uint64_t>(s1a) + (h ? run0 + (excl >> 16) : (excl & 0xffff));
        const uint64_t wb = (r >> 1) & ~uint64_t{7};
        wbase[i][h] = wb;
        rank0[i][h] = static_cast<uint32_t>(r - 2 * wb);
        win[i][h] = u32x2{0, 0};
        if (g0 + i < groups && (h ? m1 : m0) && wb + 8 <= y_bytes)
          win[i][h] = *reinterpret_cast<const u32x2 *>(Y + wb);
      }
    }
    // phase 3: words
#pragma unroll
    for (int i = 0; i < F; ++i) {
      const uint64_t g = g0 + i;
      if (g >= groups) break;
      uint32_t ex[2][2];
      const uint32_t all3 = pw[i][0] & pw[i][1] & pw[i][2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          uint32_t codes = 0;
#pragma unroll
          for (int k = 0; k < 3; ++k) codes |= ((((pw[i][k] >> (8 * h + 4 * q)) & 0xf) * 0x00204081u) & 0x01010101u) << k;
          ex[h][q] = __builtin_amdgcn_perm(t1_hi, t1_lo, codes);
        }
        uint32_t m = (all3 >> (8 * h)) & 0xff;
        uint32_t q = rank0[i][h];
        while (m) {
          const int j = __builtin_ctz(m);
          m &= m - 1;
          uint32_t yb;
          if (q < 16 && wbase[i][h] + 8 <= y_bytes) {
            yb = (q < 8 ? win[i][h].x : win[i][h].y) >> (4 * (q & 7));
          } else {
            const uint64_t byte = wbase[i][h] + (q >> 1);
            yb = byte < y_bytes ? static_cast<uint32_t>(Y[byte]) >> (4 * (q & 1)) : 0u;
          }
          const uint32_t c2 = yb & 0xf;
          const uint32_t e = __builtin_amdgcn_perm(c2 < 8 ? t2a_hi : t2b_hi, c2 < 8 ? t2a_lo : t2b_lo, c2 & 7) & 0xff;
          const uint32_t sh = 8 * (j & 3);
          if (j < 4)
            ex[h][0] = (ex[h][0] & ~(0xffu << sh)) | (e << sh);
          else
            ex[h][1] = (ex[h][1] & ~(0xffu << sh)) | (e << sh);
          ++q;
        }
      }
      const uint32_t s2a = __shfl(s2v, i, 64);
      const uint32_t s2b = min(static_cast<uint64_t>(__shfl(s2v, i + 1, 64)), e2);
      for (uint32_t k = s2a; k < s2b; ++k) {  // wave-uniform; secondary escapes are rarer still
        const uint32_t x = X[k];
        const uint32_t pos = x >> 8;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (pos == static_cast<uint32_t>(512 * h + 8 * lane + j))
              ex[h][j >> 2] = (ex[h][j >> 2] & ~(0xffu << (8 * (j & 3)))) | ((x & 0xffu) << (8 * (j & 3)));
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint64_t w0 = g * kExpcodeGroupWords + 512 * h + 8 * static_cast<uint64_t>(lane);
        uint8_t *out = dst + 2 * w0;
        u32x4 v;
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const uint32_t sel = half ? 0x0c030c02u : 0x0c010c00u;
            const uint32_t av = __builtin_amdgcn_perm(0u, a[i][h][q], sel);
            const uint32_t ev = __builtin_amdgcn_perm(0u, ex[h][q], sel);
            v[2 * q + half] = ((av & 0x00800080u) << 8) | (ev << 7) | (av & 0x007f007fu);
          }
        if (w0 + 8 <= n_words) {
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(out));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (w0 + j < n_words) reinterpret_cast<uint16_t *>(out)[j] = static_cast<uint16_t>(v[j >> 1] >> (16 * (j & 1)));
        }
      }
    }
  }
}

}  // namespace

hipError_t allow_expcode_lds(size_t bytes) {
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(expcode_decode_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute(reinterpret_cast<const void *>(expcode_dense_link_decode_kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

hipError_t launch_expcode_decode(void *dst, const void *src_dev, uint64_t capacity, uint64_t n, int grid,
                                 size_t reserve_lds, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const uint64_t groups = (n / 2 + kExpcodeGroupWords - 1) / kExpcodeGroupWords;
  const uint64_t per_block = static_cast<uint64_t>(kExpWaves) * kExpInFlight;
  const uint64_t need = std::max<uint64_t>(1, (groups + per_block - 1) / per_block);
  const unsigned g = static_cast<unsigned>(std::max<uint64_t>(1, std::min<uint64_t>(need, static_cast<uint64_t>(grid))));
  hipLaunchKernelGGL(expcode_decode_kernel, dim3(g), dim3(kExpThreads), static_cast<unsigned>(reserve_lds), stream,
                     static_cast<uint8_t *>(dst), static_cast<const uint8_t *>(src_dev), capacity, n);
  return hipGetLastError();
}

hipError_t launch_expcode_dense_link_decode(void *dst, const void *src_dev, uint64_t capacity, uint64_t n, int grid,
                                            size_t reserve_lds, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const uint64_t groups = (n / 2 + kExpcodeGroupWords - 1) / kExpcodeGroupWords;
  const uint64_t per_block = static_cast<uint64_t>(kExpWaves) * kDenseLinkInFlight;
  const uint64_t need = std::max<uint64_t>(1, (groups + per_block - 1) / per_block);
  const unsigned g = static_cast<unsigned>(std::max<uint64_t>(1, std::min<uint64_t>(need, static_cast<uint64_t>(grid))));
  hipLaunchKernelGGL(expcode_dense_link_decode_kernel, dim3(g), dim3(kExpThreads), static_cast<unsigned>(reserve_lds),
                     stream, static_cast<uint8_t *>(dst), static_cast<const uint8_t *>(src_dev), capacity, n);
  return hipGetLastError();
}

hipError_t launch_expcode_dense_decode(void *dst, const void *src_dev, uint64_t capacity, uint64_t n, int grid,
                                       size_t reserve_lds, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const uint64_t groups = (n / 2 + kExpcodeGroupWords - 1) / kExpcodeGroupWords;
  const uint64_t per_block = static_cast<uint64_t>(kExpWaves) * kDenseInFlight;
  const uint64_t need = std::max<uint64_t>(1, (groups + per_block - 1) / per_block);
  const unsigned g = static_cast<unsigned>(std::max<uint64_t>(1, std::min<uint64_t>(need, static_cast<uint64_t>(grid))));
  hipLaunchKernelGGL(expcode_dense_decode_kernel, dim3(g), dim3(kExpThreads), static_cast<unsigned>(reserve_lds),
                     stream, static_cast<uint8_t *>(dst), static_cast<const uint8_t *>(src_dev), capacity, n);
  return hipGetLastError();
}

}  // namespace ftx
