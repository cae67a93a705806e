// Philox4x32-10, BLAKE3 and the draws built on them. See rng.h for the reference each follows.
#include "rng.h"

#include <cmath>
#include <cstring>
#include <stdexcept>

namespace msx {

Philox4 philox4x32_10(const uint32_t counter[4], const uint32_t key[2]) {
  // Salmon et al., SC 2011: ten rounds, the key bumped by the Weyl constants between rounds.
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  uint32_t c0 = counter[0], c1 = counter[1], c2 = counter[2], c3 = counter[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int round = 0; round < 10; ++round) {
    if (round > 0) { k0 += W0; k1 += W1; }
    uint64_t p0 = uint64_t(M0) * c0, p1 = uint64_t(M1) * c2;
    uint32_t hi0 = uint32_t(p0 >> 32), lo0 = uint32_t(p0), hi1 = uint32_t(p1 >> 32), lo1 = uint32_t(p1);
    uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
  }
  return Philox4{{c0, c1, c2, c3}};
}

Philox4 philox_block(uint64_t seed, Stream stream, uint64_t id, uint32_t index) {
  uint32_t counter[4] = {index, uint32_t(stream), uint32_t(id), uint32_t(id >> 32)};
  uint32_t key[2] = {uint32_t(seed), uint32_t(seed >> 32)};
  return philox4x32_10(counter, key);
}

double uniform_word(uint32_t w) { return (double(w) + 0.5) / 4294967296.0; }

// ---------------------------------------------------------------------------------------------
// BLAKE3 (O'Connor, Aumasson, Neves, Wilcox-O'Hearn, 2020), default hash mode, 32-byte output.
namespace {
const uint32_t kIV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                         0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
const int kPerm[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
enum : uint32_t { CHUNK_START = 1, CHUNK_END = 2, PARENT = 4, ROOT = 8 };

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

inline void g(uint32_t* s, int a, int b, int c, int d, uint32_t x, uint32_t y) {
  s[a] = s[a] + s[b] + x; s[d] = rotr(s[d] ^ s[a], 16);
  s[c] = s[c] + s[d];     s[b] = rotr(s[b] ^ s[c], 12);
  s[a] = s[a] + s[b] + y; s[d] = rotr(s[d] ^ s[a], 8);
  s[c] = s[c] + s[d];     s[b] = rotr(s[b] ^ s[c], 7);
}

void compress(const uint32_t cv[8], const uint32_t block[16], uint64_t counter, uint32_t len,
              uint32_t flags, uint32_t out[16]) {
  uint32_t s[16] = {cv[0], cv[1], cv[2], cv[3], cv[4], cv[5], cv[6], cv[7],
                    kIV[0], kIV[1], kIV[2], kIV[3], uint32_t(counter), uint32_t(counter >> 32), len, flags};
  uint32_t m[16];
  std::memcpy(m, block, sizeof m);
  for (int r = 0; r < 7; ++r) {
    g(s, 0, 4, 8, 12, m[0], m[1]);   g(s, 1, 5, 9, 13, m[2], m[3]);
    g(s, 2, 6, 10, 14, m[4], m[5]);  g(s, 3, 7, 11, 15, m[6], m[7]);
    g(s, 0, 5, 10, 15, m[8], m[9]);  g(s, 1, 6, 11, 12, m[10], m[11]);
    g(s, 2, 7, 8, 13, m[12], m[13]); g(s, 3, 4, 9, 14, m[14], m[15]);
    if (r < 6) {
      uint32_t t[16];
      for (int i = 0; i < 16; ++i) t[i] = m[kPerm[i]];
      std::memcpy(m, t, sizeof m);
    }
  }
  for (int i = 0; i < 8; ++i) { out[i] = s[i] ^ s[i + 8]; out[i + 8] = s[i + 8] ^ cv[i]; }
}

void load_block(const uint8_t* p, size_t n, uint32_t block[16]) {
  uint8_t buf[64] = {0};
  std::memcpy(buf, p, n);
  for (int i = 0; i < 16; ++i)
    block[i] = uint32_t(buf[4 * i]) | uint32_t(buf[4 * i + 1]) << 8 | uint32_t(buf[4 * i + 2]) << 16 |
               uint32_t(buf[4 * i + 3]) << 24;
}

// The chaining value of chunk `index` (up to 1024 bytes), with `root` set on its last block
// when the chunk is the whole input.
void chunk_cv(const uint8_t* p, size_t n, uint64_t index, bool root, uint32_t cv[8]) {
  std::memcpy(cv, kIV, sizeof kIV);
  size_t blocks = n == 0 ? 1 : (n + 63) / 64;
  for (size_t b = 0; b < blocks; ++b) {
    size_t len = (b + 1 == blocks) ? n - 64 * b : 64;
    uint32_t block[16];
    load_block(p + 64 * b, len, block);
    uint32_t flags = (b == 0 ? uint32_t(CHUNK_START) : 0u) | (b + 1 == blocks ? uint32_t(CHUNK_END) : 0u);
    if (root && b + 1 == blocks) flags |= ROOT;
    uint32_t out[16];
    compress(cv, block, index, uint32_t(len), flags, out);
    std::memcpy(cv, out, 8 * sizeof(uint32_t));
  }
}

// The chaining value of the subtree over chunks [first, first + count).
void subtree_cv(const uint8_t* data, size_t len, uint64_t first, uint64_t count, bool root, uint32_t cv[8]) {
  if (count == 1) {
    size_t start = size_t(first) * 1024;
    size_t n = len - start < 1024 ? len - start : 1024;
    chunk_cv(data + start, n, first, root, cv);
    return;
  }
  uint64_t left = 1;
  while (left * 2 < count) left *= 2;  // largest power of two below count
  uint32_t block[16];
  subtree_cv(data, len, first, left, false, block);
  subtree_cv(data, len, first + left, count - left, false, block + 8);
  uint32_t out[16];
  compress(kIV, block, 0, 64, uint32_t(PARENT) | (root ? uint32_t(ROOT) : 0u), out);
  std::memcpy(cv, out, 8 * sizeof(uint32_t));
}
}  // namespace

void blake3(const void* data, size_t len, uint8_t out[32]) {
  uint64_t chunks = len == 0 ? 1 : (len + 1023) / 1024;
  uint32_t cv[8];
  subtree_cv(static_cast<const uint8_t*>(data), len, 0, chunks, true, cv);
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 4; ++j) out[4 * i + j] = uint8_t(cv[i] >> (8 * j));
}

static uint64_t first8_le(const uint8_t h[32]) {
  uint64_t v = 0;
  for (int i = 7; i >= 0; --i) v = (v << 8) | h[i];
  return v;
}

uint64_t canonical_id(const std::string& path) {
  uint8_t h[32];
  blake3(path.data(), path.size(), h);
  return first8_le(h);
}

uint64_t dropout_id(const std::string& site, uint64_t step) {
  std::string bytes = site;
  for (int i = 0; i < 8; ++i) bytes.push_back(char(uint8_t(step >> (8 * i))));
  uint8_t h[32];
  blake3(bytes.data(), bytes.size(), h);
  return first8_le(h);
}

void dropout_token(const std::string& site, uint64_t step, int32_t out[2]) {
  uint64_t id = dropout_id(site, step);
  out[0] = int32_t(uint32_t(id));
  out[1] = int32_t(uint32_t(id >> 32));
}

bool dropout_keeps(uint64_t seed, uint64_t id, uint32_t index, float p) {
  return uniform_word(philox_block(seed, Stream::Dropout, id, index).w[0]) >= double(p);
}

uint64_t dropout_threshold(float p) {
  // (w + 0.5)/2^32 >= p  <=>  w >= p*2^32 - 0.5, every step exact in f64 for p in [0, 1).
  double x = double(p) * 4294967296.0 - 0.5;
  if (x <= 0) return 0;
  return uint64_t(std::ceil(x));
}

std::vector<float> xavier_uniform(uint64_t seed, Stream stream, const std::string& path, int64_t fan_in,
                                  int64_t fan_out) {
  double a = std::sqrt(6.0 / (double(fan_in) + double(fan_out)));
  uint64_t id = canonical_id(path);
  int64_t n = fan_in * fan_out;
  std::vector<float> v(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) {
    uint32_t w = philox_block(seed, stream, id, uint32_t(i)).w[0];
    v[size_t(i)] = float(a * (2.0 * uniform_word(w) - 1.0));
  }
  return v;
}

std::vector<float> standard_normal(uint64_t seed, Stream stream, const std::string& name, int64_t count) {
  uint64_t id = canonical_id(name);
  std::vector<float> v(static_cast<size_t>(count));
  const double tau = 6.283185307179586;
  for (int64_t i = 0; i < count; ++i) {
    Philox4 b = philox_block(seed, stream, id, uint32_t(i));
    v[size_t(i)] = float(std::sqrt(-2.0 * std::log(uniform_word(b.w[0]))) * std::cos(tau * uniform_word(b.w[1])));
  }
  return v;
}

double powi(double a, int b) {
  const bool recip = b < 0;
  double r = 1;
  while (true) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1 / r : r;
}

}  // namespace msx
