/*
 * CPU oracle for the byte-level parts of the weight-streaming path.
 * TEST INFRASTRUCTURE ONLY: tests, the smoke check and the CPU-baseline leg of
 * bench.py may load this library as the checker; the product never does.
 *
 *   oracle_packed_layout  follows _compute_packed_byte_layout (utils.py:114-127):
 *                         offset_i = cursor; cursor = ceil_align(cursor + size_i).
 *   oracle_pack           follows AllocationBlock._tensors_to_memory_block
 *                         (allocation_block.py:179-181): per-tensor byte copy of a
 *                         dense tensor's storage bytes into the block at its offset.
 *                         Pinned by the reference's three-tensor block and its
 *                         Fortran byte-order case (test_allocation_block.py:14-56,
 *                         test_stride_preservation.py:38-70), written out byte
 *                         by byte; a shifted offset fails that check.
 *   oracle_scatter        the semantics of one batched scatter: for every
 *                         descriptor dst[0:n) = chunk[off:off+n), as the
 *                         reference's per-tensor copies produce it
 *                         (allocation_block.py:104-106, loaders.py:1064-1067).
 *   oracle_checksum64     the checksum definition the device checksum must match.
 */
#include <stdint.h>
#include <string.h>
#include <stddef.h>

typedef struct oracle_desc {
  uint64_t src_off;
  uint64_t dst; /* host address of the destination buffer */
  uint64_t nbytes;
} oracle_desc;

uint64_t oracle_packed_layout(const uint64_t *sizes, int n, uint64_t alignment, uint64_t *offsets) {
  uint64_t cursor = 0;
  for (int i = 0; i < n; ++i) {
    offsets[i] = cursor;
    cursor += sizes[i];
    cursor = (cursor + alignment - 1) / alignment * alignment;
  }
  return cursor;
}

void oracle_pack(uint8_t *block, const uint64_t *offsets, const uint64_t *srcs, const uint64_t *sizes, int n) {
  for (int i = 0; i < n; ++i) memcpy(block + offsets[i], (const void *)(uintptr_t)srcs[i], (size_t)sizes[i]);
}

void oracle_scatter(const uint8_t *chunk, const oracle_desc *descs, int n) {
  for (int i = 0; i < n; ++i)
    memcpy((void *)(uintptr_t)descs[i].dst, chunk + descs[i].src_off, (size_t)descs[i].nbytes);
}

static uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

/* Word w (8 bytes little-endian, zero padded past n) belongs to block w/512,
 * lane (w%512)%64, step (w%512)/64. Lane hash: FNV-1a over 64-bit words.
 * block_sum = sum over lanes of splitmix64(h + lane);
 * result = splitmix64(sum over blocks of splitmix64(block_sum + block) + n). */
uint64_t oracle_checksum64(const uint8_t *p, uint64_t n) {
  const uint64_t n_blocks = (n + 4095) / 4096;
  uint64_t total = 0;
  for (uint64_t b = 0; b < n_blocks; ++b) {
    uint64_t block_sum = 0;
    for (uint64_t lane = 0; lane < 64; ++lane) {
      uint64_t h = 0xcbf29ce484222325ull;
      for (uint64_t k = 0; k < 8; ++k) {
        const uint64_t w = b * 512 + k * 64 + lane;
        uint64_t x = 0;
        if (w * 8 + 8 <= n) {
          memcpy(&x, p + w * 8, 8);
        } else if (w * 8 < n) {
          for (uint64_t q = w * 8; q < n; ++q) x |= (uint64_t)p[q] << (8 * (q - w * 8));
        }
        h = (h ^ x) * 0x100000001b3ull;
      }
      block_sum += splitmix64(h + lane);
    }
    total += splitmix64(block_sum + b);
  }
  return splitmix64(total + n);
}
