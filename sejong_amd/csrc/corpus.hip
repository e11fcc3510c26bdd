// Corpus fingerprint: BLAKE3 (the `blake3` crate 1.8.7 of the reference's
// Cargo.lock, used by Corpus::open, crates/sejong-train/src/lib.rs:32-56),
// written from the published BLAKE3 specification (O'Connor, Aumasson,
// Neves, Wilcox-O'Hearn, 2020): 32-bit words, the compression function of 7
// rounds over a 4 x 4 state with the message permutation between rounds,
// 1024-byte chunks of 64-byte blocks, chunk chaining values merged into a
// binary tree of parent nodes as chunks complete, and the root node's output
// as the 32-byte hash (default hash mode: key = IV, no flags beyond the
// node flags).  Host code only; the caller owns the hasher state.
#include <stdint.h>
#include <string.h>

#include "common.h"

namespace {

constexpr uint32_t IV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                            0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
constexpr int PERM[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
constexpr uint32_t CHUNK_START = 1, CHUNK_END = 2, PARENT = 4, ROOT = 8;
constexpr size_t BLOCK = 64, CHUNK = 1024;
constexpr int MAX_DEPTH = 54;  // chunks of 2^10 bytes, inputs below 2^64 bytes

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

inline void g(uint32_t* s, int a, int b, int c, int d, uint32_t mx, uint32_t my) {
  s[a] = s[a] + s[b] + mx;
  s[d] = rotr(s[d] ^ s[a], 16);
  s[c] = s[c] + s[d];
  s[b] = rotr(s[b] ^ s[c], 12);
  s[a] = s[a] + s[b] + my;
  s[d] = rotr(s[d] ^ s[a], 8);
  s[c] = s[c] + s[d];
  s[b] = rotr(s[b] ^ s[c], 7);
}

// the compression function: 16 output words of (chaining value, block,
// counter, block length, flags)
void compress(const uint32_t cv[8], const uint32_t block[16], uint64_t counter, uint32_t len, uint32_t flags,
              uint32_t out[16]) {
  uint32_t s[16] = {cv[0], cv[1], cv[2], cv[3], cv[4], cv[5], cv[6], cv[7],
                    IV[0], IV[1], IV[2], IV[3], (uint32_t)counter, (uint32_t)(counter >> 32), len, flags};
  uint32_t m[16];
  memcpy(m, block, sizeof(m));
  for (int r = 0; r < 7; r++) {
    g(s, 0, 4, 8, 12, m[0], m[1]);  // columns
    g(s, 1, 5, 9, 13, m[2], m[3]);
    g(s, 2, 6, 10, 14, m[4], m[5]);
    g(s, 3, 7, 11, 15, m[6], m[7]);
    g(s, 0, 5, 10, 15, m[8], m[9]);  // diagonals
    g(s, 1, 6, 11, 12, m[10], m[11]);
    g(s, 2, 7, 8, 13, m[12], m[13]);
    g(s, 3, 4, 9, 14, m[14], m[15]);
    if (r < 6) {
      uint32_t p[16];
      for (int i = 0; i < 16; i++) p[i] = m[PERM[i]];
      memcpy(m, p, sizeof(m));
    }
  }
  for (int i = 0; i < 8; i++) {
    out[i] = s[i] ^ s[i + 8];
    out[i + 8] = s[i + 8] ^ cv[i];
  }
}

void words_le(const uint8_t* b, uint32_t w[16]) {
  for (int i = 0; i < 16; i++)
    w[i] = (uint32_t)b[4 * i] | ((uint32_t)b[4 * i + 1] << 8) | ((uint32_t)b[4 * i + 2] << 16) |
           ((uint32_t)b[4 * i + 3] << 24);
}

// a node whose chaining value or root output is still to be taken
struct Node {
  uint32_t cv[8];
  uint32_t block[16];
  uint64_t counter;
  uint32_t len, flags;
  void chaining_value(uint32_t out[8]) const {
    uint32_t w[16];
    compress(cv, block, counter, len, flags, w);
    memcpy(out, w, 32);
  }
};

Node parent(const uint32_t left[8], const uint32_t right[8]) {
  Node n;
  memcpy(n.cv, IV, 32);
  memcpy(n.block, left, 32);
  memcpy(n.block + 8, right, 32);
  n.counter = 0;
  n.len = BLOCK;
  n.flags = PARENT;
  return n;
}

struct Hasher {
  // the chunk being filled
  uint32_t cv[8];
  uint64_t chunk;  // its index
  uint8_t block[BLOCK];
  uint32_t block_len, blocks_done;
  // chaining values of completed subtrees, largest first
  uint32_t stack[MAX_DEPTH][8];
  int depth;
  uint64_t magic;

  void start_chunk(uint64_t index) {
    memcpy(cv, IV, 32);
    chunk = index;
    memset(block, 0, sizeof(block));
    block_len = 0;
    blocks_done = 0;
  }
  uint32_t start_flag() const { return blocks_done == 0 ? CHUNK_START : 0; }
  size_t chunk_len() const { return (size_t)blocks_done * BLOCK + block_len; }
  Node chunk_output() const {
    Node n;
    memcpy(n.cv, cv, 32);
    words_le(block, n.block);
    n.counter = chunk;
    n.len = block_len;
    n.flags = start_flag() | CHUNK_END;
    return n;
  }
  // a completed chunk's chaining value joins the tree: merge it with the
  // stacked subtrees while the completed-chunk count has trailing zeros
  void push_chunk(uint32_t value[8], uint64_t total) {
    uint32_t v[8];
    memcpy(v, value, 32);
    while ((total & 1) == 0) {
      parent(stack[--depth], v).chaining_value(v);
      total >>= 1;
    }
    memcpy(stack[depth++], v, 32);
  }
  void update(const uint8_t* p, size_t n) {
    while (n > 0) {
      if (chunk_len() == CHUNK) {
        uint32_t v[8];
        chunk_output().chaining_value(v);
        const uint64_t total = chunk + 1;
        push_chunk(v, total);
        start_chunk(total);
      }
      // fill the chunk's blocks; a full block is compressed only once more
      // input follows (the chunk's last block carries CHUNK_END)
      size_t take = CHUNK - chunk_len();
      if (take > n) take = n;
      while (take > 0) {
        if (block_len == BLOCK) {
          uint32_t w[16], out[16];
          words_le(block, w);
          compress(cv, w, chunk, BLOCK, start_flag(), out);
          memcpy(cv, out, 32);
          blocks_done++;
          memset(block, 0, sizeof(block));
          block_len = 0;
        }
        size_t k = BLOCK - block_len;
        if (k > take) k = take;
        memcpy(block + block_len, p, k);
        block_len += (uint32_t)k;
        p += k;
        n -= k;
        take -= k;
      }
    }
  }
  void finalize(uint8_t out[32]) const {
    Node n = chunk_output();
    for (int i = depth - 1; i >= 0; i--) {
      uint32_t v[8];
      n.chaining_value(v);
      n = parent(stack[i], v);
    }
    uint32_t w[16];
    compress(n.cv, n.block, 0, n.len, n.flags | ROOT, w);
    for (int i = 0; i < 8; i++)
      for (int b = 0; b < 4; b++) out[4 * i + b] = (uint8_t)(w[i] >> (8 * b));
  }
};

constexpr uint64_t MAGIC = 0x4233484153484552ull;

}  // namespace

extern "C" size_t sj_blake3_state_bytes(void) { return sizeof(Hasher); }

extern "C" int sj_blake3_init(void* state) {
  SJ_REQUIRE(state, "blake3: null state");
  Hasher* h = (Hasher*)state;
  memset(h, 0, sizeof(*h));
  h->start_chunk(0);
  h->depth = 0;
  h->magic = MAGIC;
  return SJ_OK;
}

extern "C" int sj_blake3_update(void* state, const void* data, size_t bytes) {
  SJ_REQUIRE(state && ((Hasher*)state)->magic == MAGIC && (data || bytes == 0), "blake3: update arguments");
  ((Hasher*)state)->update((const uint8_t*)data, bytes);
  return SJ_OK;
}

extern "C" int sj_blake3_finalize(const void* state, uint8_t* out32) {
  SJ_REQUIRE(state && ((const Hasher*)state)->magic == MAGIC && out32, "blake3: finalize arguments");
  ((const Hasher*)state)->finalize(out32);
  return SJ_OK;
}
