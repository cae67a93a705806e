// Counter-based random draws and path hashing shared by the host runtime and its tests.
//
// Restates crates/modelspec-runtime/src/train/init.rs:91-165 (Philox4x32-10, canonical ids,
// dropout ids and tokens, the dropout keep rule) and the BLAKE3 hash those ids are built on
// (blake3 1.8.7, Cargo.lock:165; the published BLAKE3 specification).
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace msx {

// Stream tags of the Philox counter (init.rs:46-77).
enum class Stream : uint32_t { Init = 0, Teacher = 1, Data = 2, Masking = 3, Dropout = 4, DataOrder = 5, Projection = 6 };

struct Philox4 { uint32_t w[4]; };

// Philox4x32-10 of `counter` under `key` (init.rs:91-109).
Philox4 philox4x32_10(const uint32_t counter[4], const uint32_t key[2]);

// The block of element `index` of draw `id` on `stream` under `seed` (init.rs:120-126).
Philox4 philox_block(uint64_t seed, Stream stream, uint64_t id, uint32_t index);

// (w + 0.5) / 2^32 in f64 (init.rs:129-131).
double uniform_word(uint32_t w);

// BLAKE3 of `data` (32-byte digest), the default hash mode.
void blake3(const void* data, size_t len, uint8_t out[32]);

// First 8 bytes of blake3(path), little-endian (init.rs:112-118).
uint64_t canonical_id(const std::string& path);

// First 8 bytes of blake3(site ‖ step as u64 LE), little-endian (init.rs:133-143).
uint64_t dropout_id(const std::string& site, uint64_t step);

// The i32[2] token [low, high] of dropout_id (init.rs:145-151).
void dropout_token(const std::string& site, uint64_t step, int32_t out[2]);

// The draw id a token holds (init.rs:153-156).
inline uint64_t token_id(const int32_t token[2]) {
  return uint64_t(uint32_t(token[0])) | (uint64_t(uint32_t(token[1])) << 32);
}

// Kept iff uniform(word 0 of the Dropout block) >= p, compared in f64 (init.rs:158-165).
bool dropout_keeps(uint64_t seed, uint64_t id, uint32_t index, float p);

// The smallest word w with (w + 0.5)/2^32 >= p: element kept iff word0 >= threshold. The
// comparison is exact in f64, so the integer threshold decides the same bits on the device.
uint64_t dropout_threshold(float p);

// xavier_uniform of a [fan_in, fan_out] tensor (init.rs:197-222).
std::vector<float> xavier_uniform(uint64_t seed, Stream stream, const std::string& path,
                                  int64_t fan_in, int64_t fan_out);

// Box-Muller standard normal draw of `count` elements named `name` (init.rs:224-234).
std::vector<float> standard_normal(uint64_t seed, Stream stream, const std::string& name, int64_t count);

// compiler-rt __powidf2: repeated squaring, the lowering of Rust's f64::powi.
double powi(double a, int b);

}  // namespace msx
