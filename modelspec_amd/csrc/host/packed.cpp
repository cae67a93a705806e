// The packed data path of packed.h.
#include "packed.h"

#include <sys/stat.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>

#include "json.h"
#include "rng.h"

namespace msx {
namespace {

const char* kBinding = "binding.json";
const char* kPacked = "packed.json";
const char* kTrainTokens = "train.tokens";
const char* kHeldOutTokens = "heldout.tokens";

std::string join(const std::string& dir, const std::string& file) {
  return dir.empty() || dir.back() == '/' ? dir + file : dir + "/" + file;
}

[[noreturn]] void refuse(const std::string& path, const std::string& why) { throw PackedError(path + ": " + why); }

std::string read_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) refuse(path, std::string("cannot be read (") + std::strerror(errno) + ")");
  std::ostringstream s;
  s << f.rdbuf();
  return s.str();
}

void write_file(const std::string& path, const void* data, size_t bytes) {
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) refuse(path, std::string("cannot be written (") + std::strerror(errno) + ")");
  f.write(static_cast<const char*>(data), std::streamsize(bytes));
  if (!f) refuse(path, "a short write");
}

std::string hex(const uint8_t* b, size_t n) {
  static const char* d = "0123456789abcdef";
  std::string s;
  for (size_t i = 0; i < n; ++i) {
    s += d[b[i] >> 4];
    s += d[b[i] & 15];
  }
  return s;
}

// The 16 bytes of a hyphenated UUID (mlm.rs:147-159); false when `text` is not one.
bool uuid_bytes(const std::string& text, uint8_t out[16]) {
  if (text.size() != 36) return false;
  std::string h;
  for (char c : text)
    if (c != '-') h += c;
  if (h.size() != 32) return false;
  for (int i = 0; i < 16; ++i) {
    unsigned v = 0;
    for (int k = 0; k < 2; ++k) {
      char c = h[size_t(2 * i + k)];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= unsigned(c - '0');
      else if (c >= 'a' && c <= 'f') v |= unsigned(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= unsigned(c - 'A' + 10);
      else return false;
    }
    out[i] = uint8_t(v);
  }
  return true;
}

void put_u64(std::string& s, uint64_t v) {
  for (int k = 0; k < 8; ++k) s += char(uint8_t(v >> (8 * k)));
}

// The shortest decimal text that reads back as `v` (serde_json's form of an f64).
std::string shortest(double v) {
  char buf[40];
  for (int prec = 1; prec <= 17; ++prec) {
    std::snprintf(buf, sizeof buf, "%.*g", prec, v);
    if (std::strtod(buf, nullptr) == v) break;
  }
  std::string s = buf;
  if (s.find_first_of(".eEn") == std::string::npos) s += ".0";
  return s;
}

// The smallest word w with (w + 0.5) / 2^32 >= rate; 2^32 when there is none.
uint64_t word_threshold(double rate) {
  uint64_t lo = 0, hi = uint64_t(1) << 32;
  while (lo < hi) {
    uint64_t mid = lo + (hi - lo) / 2;
    if (uniform_word(uint32_t(mid)) >= rate) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

}  // namespace

std::string uuid_of(const uint8_t hash[32]) {
  uint8_t b[16];
  std::memcpy(b, hash, 16);
  b[6] = uint8_t((b[6] & 0x0f) | 0x80);
  b[8] = uint8_t((b[8] & 0x3f) | 0x80);
  std::string h = hex(b, 16);
  return h.substr(0, 8) + "-" + h.substr(8, 4) + "-" + h.substr(12, 4) + "-" + h.substr(16, 4) + "-" + h.substr(20, 12);
}

std::string binding_id(const std::string& dataset_id, const std::string& tokenizer_id, uint64_t seq_len,
                       const MaskingPolicy& p) {
  uint8_t d[16], t[16];
  if (!uuid_bytes(dataset_id, d) || !uuid_bytes(tokenizer_id, t)) return "";
  std::string bytes(reinterpret_cast<char*>(d), 16);
  bytes.append(reinterpret_cast<char*>(t), 16);
  put_u64(bytes, seq_len);
  for (double rate : {p.selection_rate, p.mask_fraction, p.random_fraction, p.keep_fraction}) {
    uint64_t bits;
    std::memcpy(&bits, &rate, 8);
    put_u64(bytes, bits);
  }
  uint8_t h[32];
  blake3(bytes.data(), bytes.size(), h);
  return uuid_of(h);
}

MaskingThresholds masking_thresholds(const MaskingPolicy& p) {
  MaskingThresholds t;
  t.select = word_threshold(p.selection_rate);
  t.mask = word_threshold(p.mask_fraction);
  t.mask_or_random = word_threshold(p.mask_fraction + p.random_fraction);
  return t;
}

PackedCorpus load_packed(const std::string& dir) {
  PackedCorpus c;
  c.dir = dir;
  const std::string bpath = join(dir, kBinding), ppath = join(dir, kPacked);
  try {
    // The binding first, and its id against its fields (train/data.rs:1448-1482).
    json::Value b = json::parse(read_file(bpath));
    c.binding_id = b.at("binding_id").str();
    c.dataset_id = b.at("dataset_id").str();
    c.tokenizer_id = b.at("tokenizer_id").str();
    c.seq_len = b.at("seq_len").u64();
    const json::Value& pol = b.at("masking_policy");
    c.policy.selection_rate = pol.at("selection_rate").number();
    c.policy.mask_fraction = pol.at("mask_fraction").number();
    c.policy.random_fraction = pol.at("random_fraction").number();
    c.policy.keep_fraction = pol.at("keep_fraction").number();
    if (b.at("state").str() != "Recorded") refuse(bpath, "a binding whose state is not Recorded");
  } catch (const PackedError&) {
    throw;
  } catch (const std::exception& e) {
    refuse(bpath, e.what());
  }
  if (c.seq_len == 0 || binding_id(c.dataset_id, c.tokenizer_id, c.seq_len, c.policy) != c.binding_id)
    refuse(bpath, "binding_id " + c.binding_id + " is not the id of its dataset, tokenizer, seq_len and masking policy");

  // The record (mlm.rs:588-662).
  struct Split { std::string role; uint64_t count; std::string hash; };
  std::vector<Split> splits;
  std::string record_binding;
  uint64_t record_seq = 0;
  try {
    json::Value p = json::parse(read_file(ppath));
    c.packed_id = p.at("packed_id").str();
    record_binding = p.at("binding_id").str();
    record_seq = p.at("seq_len").u64();
    c.vocabulary_size = p.at("vocabulary_size").u64();
    c.heldout_unigram_baseline_nats = p.at("heldout_unigram_baseline_nats").number();
    const json::Value& s = p.at("splits");
    if (s.kind != json::Value::Array) refuse(ppath, "splits is not an array");
    for (auto& x : s.items) splits.push_back({x.at("role").str(), x.at("sequence_count").u64(), x.at("content_hash").str()});
  } catch (const PackedError&) {
    throw;
  } catch (const std::exception& e) {
    refuse(ppath, e.what());
  }
  if (splits.size() != 2 || splits[0].role != "Train" || splits[1].role != "HeldOut" || record_seq == 0)
    refuse(ppath, "not a record of a Train and a HeldOut split of a positive sequence length");
  if (c.vocabulary_size <= kSpecialTokens || c.vocabulary_size > (uint64_t(1) << 31))
    refuse(ppath, "vocabulary_size " + std::to_string(c.vocabulary_size) + " is not between 6 and 2^31");
  for (int k = 0; k < 2; ++k) {
    const std::string path = join(dir, k == 0 ? kTrainTokens : kHeldOutTokens);
    std::string bytes = read_file(path);
    const Split& s = splits[size_t(k)];
    const unsigned __int128 want = (unsigned __int128)s.count * record_seq * 4;
    if (s.count > UINT32_MAX || want != bytes.size())
      refuse(path, std::to_string(bytes.size()) + " bytes, not " + std::to_string(s.count) + " sequences of " +
                       std::to_string(record_seq) + " ids");
    uint8_t h[32];
    blake3(bytes.data(), bytes.size(), h);
    if (hex(h, 32) != s.hash) refuse(path, std::string("blake3 differs from the content_hash of ") + kPacked);
    std::vector<int32_t>& ids = k == 0 ? c.train : c.heldout;
    ids.resize(bytes.size() / 4);
    std::memcpy(ids.data(), bytes.data(), bytes.size());  // little-endian host, as the files are
    for (int32_t t : ids)
      if (t < 0 || uint64_t(t) >= c.vocabulary_size)
        refuse(path, "id " + std::to_string(t) + " outside a vocabulary of " + std::to_string(c.vocabulary_size));
  }
  // The record belongs to the binding (train/data.rs:1620-1630).
  if (record_binding != c.binding_id || record_seq != c.seq_len)
    refuse(ppath, "binding_id " + record_binding + " and seq_len " + std::to_string(record_seq) + " are not those of " +
                      kBinding);
  return c;
}

void write_packed(const std::string& dir, const std::vector<int32_t>& train, const std::vector<int32_t>& heldout,
                  uint64_t seq_len, uint64_t vocabulary_size, const std::string& dataset_id,
                  const std::string& tokenizer_id, const MaskingPolicy& policy) {
  if (seq_len == 0) refuse(dir, "a sequence length of 0");
  if (mkdir(dir.c_str(), 0755) != 0 && errno != EEXIST) refuse(dir, std::strerror(errno));
  const std::string bid = binding_id(dataset_id, tokenizer_id, seq_len, policy);
  if (bid.empty()) refuse(dir, "dataset_id or tokenizer_id is not a UUID");
  std::string digests;
  std::string split_json;
  // pack(): the Train counts of every id that is not special, then the held-out log-likelihood
  // of each held-out id under add-one smoothing (mlm.rs:460-495).
  std::vector<uint64_t> counts(size_t(vocabulary_size), 0);
  uint64_t train_total = 0, measured = 0;
  double log_sum = 0;
  for (int k = 0; k < 2; ++k) {
    const std::vector<int32_t>& ids = k == 0 ? train : heldout;
    const uint64_t sequences = ids.size() / seq_len;
    if (sequences == 0 || ids.size() % seq_len) refuse(dir, "a split that is not a positive number of whole sequences");
    for (int32_t t : ids)
      if (t < 0 || uint64_t(t) >= vocabulary_size) refuse(dir, "an id outside the vocabulary");
    const std::string path = join(dir, k == 0 ? kTrainTokens : kHeldOutTokens);
    write_file(path, ids.data(), ids.size() * 4);
    uint8_t h[32];
    blake3(ids.data(), ids.size() * 4, h);
    digests.append(reinterpret_cast<char*>(h), 32);
    if (k == 0) {
      for (int32_t t : ids)
        if (uint32_t(t) >= kSpecialTokens) {
          ++counts[size_t(t)];
          ++train_total;
        }
    } else {
      const double types = double(vocabulary_size - kSpecialTokens), den = double(train_total) + types;
      for (int32_t t : ids)
        if (uint32_t(t) >= kSpecialTokens) {
          log_sum += std::log((double(counts[size_t(t)]) + 1.0) / den);
          ++measured;
        }
    }
    split_json += std::string(k ? ",\n" : "") + "    {\n      \"role\": \"" + (k == 0 ? "Train" : "HeldOut") +
                  "\",\n      \"sequence_count\": " + std::to_string(sequences) + ",\n      \"content_hash\": \"" +
                  hex(h, 32) + "\"\n    }";
  }
  if (measured == 0) refuse(dir, "the held-out split holds no token that is not special");
  put_u64(digests, seq_len);
  uint8_t pid[32];
  blake3(digests.data(), digests.size(), pid);
  std::string binding = "{\n  \"binding_id\": " + json::quote(bid) + ",\n  \"dataset_id\": " + json::quote(dataset_id) +
                        ",\n  \"tokenizer_id\": " + json::quote(tokenizer_id) + ",\n  \"seq_len\": " +
                        std::to_string(seq_len) + ",\n  \"masking_policy\": {\n    \"selection_rate\": " +
                        shortest(policy.selection_rate) + ",\n    \"mask_fraction\": " + shortest(policy.mask_fraction) +
                        ",\n    \"random_fraction\": " + shortest(policy.random_fraction) + ",\n    \"keep_fraction\": " +
                        shortest(policy.keep_fraction) + "\n  },\n  \"state\": \"Recorded\"\n}";
  std::string packed = "{\n  \"packed_id\": " + json::quote(uuid_of(pid)) + ",\n  \"binding_id\": " + json::quote(bid) +
                       ",\n  \"seq_len\": " + std::to_string(seq_len) + ",\n  \"vocabulary_size\": " +
                       std::to_string(vocabulary_size) + ",\n  \"splits\": [\n" + split_json +
                       "\n  ],\n  \"heldout_unigram_baseline_nats\": " + shortest(-log_sum / double(measured)) +
                       ",\n  \"state\": \"Recorded\"\n}";
  write_file(join(dir, kBinding), binding.data(), binding.size());
  write_file(join(dir, kPacked), packed.data(), packed.size());
}

const char* const kDrawInput = "#draw";

std::vector<int32_t> draw_words(SplitRole role, const SequenceDraw& d) {
  std::vector<int32_t> w{role == SplitRole::Train ? 0 : 1, int32_t(uint32_t(d.draw_id)), int32_t(uint32_t(d.draw_id >> 32))};
  w.insert(w.end(), d.sequences.begin(), d.sequences.end());
  return w;
}

const char* const kBatchTensors[5] = {"ids", "positions", "key_mask", "labels", "weights"};

uint64_t bind_corpus(const Program& forward, const PackedCorpus& c) {
  const uint64_t S = c.seq_len;
  std::vector<const Node*> inputs;
  for (auto& n : forward.nodes)
    if (n.op == Op::Input) {
      bool known = false;
      for (const char* t : kBatchTensors) known = known || n.name == t;
      if (!known)
        throw IrError("E-DATA-005: the input `" + n.name +
                      "` names no tensor of the masked-language-model batch (ids, positions, key_mask, labels, weights)");
      inputs.push_back(&n);
    }
  if (inputs.empty()) throw IrError("E-DATA-005: a run on a packed directory declares no batch tensor");
  const Node* first = nullptr;
  for (const char* t : kBatchTensors)
    if (!first)
      for (const Node* n : inputs)
        if (n->name == t) first = n;
  uint64_t B = 0;
  const auto& fs = first->ty.shape;
  if (fs.size() == 2 && fs[1] > 0 && uint64_t(fs[1]) == S && fs[0] > 0) B = uint64_t(fs[0]);
  else if (fs.size() == 1 && fs[0] > 0 && uint64_t(fs[0]) % S == 0) B = uint64_t(fs[0]) / S;
  if (B == 0)
    throw IrError("E-DATA-006: `" + first->name + "` is " + type_string(first->ty) + ", not [B, " + std::to_string(S) +
                  "] or [B*" + std::to_string(S) + "]");
  for (const Node* n : inputs) {
    const bool is_f32 = n->name == "key_mask" || n->name == "weights";
    const auto& sh = n->ty.shape;
    const bool shaped = (sh.size() == 2 && uint64_t(sh[0]) == B && uint64_t(sh[1]) == S) ||
                        (sh.size() == 1 && uint64_t(sh[0]) == B * S);
    if ((n->ty.dtype == DType::F32) != is_f32 || !shaped)
      throw IrError("E-DATA-006: `" + n->name + "` is " + type_string(n->ty) + ", not Tensor<" +
                    (is_f32 ? "f32" : "i32") + ", [" + std::to_string(B) + ", " + std::to_string(S) + "]> or [" +
                    std::to_string(B * S) + "]");
  }
  // The vocabulary the ids index and the labels classify (refuse_vocabulary).
  const Node* ids = forward.input("ids");
  const Node* labels = forward.input("labels");
  for (auto& n : forward.nodes) {
    if (n.op == Op::Embedding && ids && n.operands[1] == ids->id) {
      const Node& table = forward.node(n.operands[0]);
      if (uint64_t(table.ty.shape[0]) != c.vocabulary_size)
        throw IrError("E-DATA-006: the embedding table the ids index has " + std::to_string(table.ty.shape[0]) +
                      " rows, not the vocabulary_size " + std::to_string(c.vocabulary_size));
    }
    if (n.op == Op::CrossEntropy && labels && n.operands[1] == labels->id) {
      const Node& logits = forward.node(n.operands[0]);
      if (uint64_t(logits.ty.shape[1]) != c.vocabulary_size)
        throw IrError("E-DATA-006: the logits the labels classify have " + std::to_string(logits.ty.shape[1]) +
                      " classes, not the vocabulary_size " + std::to_string(c.vocabulary_size));
    }
  }
  if (B > c.sequences(SplitRole::Train))
    throw PackedError(c.dir + ": a batch of " + std::to_string(B) + " sequences, more than the " +
                      std::to_string(c.sequences(SplitRole::Train)) + " of the Train split");
  return B;
}

std::vector<uint32_t> epoch_order(uint64_t seed, uint64_t epoch, uint32_t n) {
  std::vector<std::pair<uint64_t, uint32_t>> keyed(n);
  for (uint32_t i = 0; i < n; ++i) {
    Philox4 w = philox_block(seed, Stream::DataOrder, epoch, i);
    keyed[i] = {(uint64_t(w.w[1]) << 32) | uint64_t(w.w[0]), i};
  }
  std::sort(keyed.begin(), keyed.end());
  std::vector<uint32_t> out(n);
  for (uint32_t i = 0; i < n; ++i) out[i] = keyed[i].second;
  return out;
}

SequenceDraw EpochOrders::draw(const PackedCorpus& c, SplitRole role, uint64_t seed, uint64_t step, uint64_t batch) {
  const uint64_t sequences = c.sequences(role);
  if (batch == 0) throw PackedError(c.dir + ": a batch of 0 sequences");
  if (batch > sequences)
    throw PackedError(c.dir + ": a batch of " + std::to_string(batch) + " sequences, more than the " +
                      std::to_string(sequences) + " of the split");
  if ((unsigned __int128)batch * c.seq_len > ((unsigned __int128)1 << 32))
    throw PackedError(c.dir + ": a batch of more than 2^32 rows");
  const uint64_t per_epoch = sequences / batch, b = step % per_epoch;
  SequenceDraw d;
  d.sequences.resize(size_t(batch));
  if (role == SplitRole::Train) {
    const uint64_t epoch = step / per_epoch;
    if (!have_ || seed_ != seed || epoch_ != epoch || order_.size() != sequences) {
      order_ = epoch_order(seed, epoch, uint32_t(sequences));
      seed_ = seed;
      epoch_ = epoch;
      have_ = true;
    }
    for (uint64_t i = 0; i < batch; ++i) d.sequences[size_t(i)] = int32_t(order_[size_t(b * batch + i)]);
    d.draw_id = step;
  } else {
    for (uint64_t i = 0; i < batch; ++i) d.sequences[size_t(i)] = int32_t(b * batch + i);
    d.draw_id = step + (uint64_t(1) << 63);
  }
  return d;
}

}  // namespace msx
