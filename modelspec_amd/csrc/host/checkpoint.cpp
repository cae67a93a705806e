// The .msckpt checkpoint of checkpoint.h.
#include "checkpoint.h"

#include <sys/stat.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <sstream>

#include "json.h"
#include "packed.h"
#include "rng.h"

namespace msx {
namespace {

constexpr size_t kHeader = 56;
constexpr uint64_t kAlign = 64;
constexpr uint32_t kVersion = 1, kEndian = 0x01020304;
constexpr size_t kMaxRank = 8;
// One record's size in the reference reader's memory, which bounds how many records a file of a
// given size may declare (checkpoint.rs:300-306, 745-750).
constexpr uint64_t kRecordBytes = 96, kSlack = 4096;
const char* kNilUuid = "00000000-0000-0000-0000-000000000000";

std::string hexs(const uint8_t* b, size_t n) {
  static const char* d = "0123456789abcdef";
  std::string s;
  for (size_t i = 0; i < n; ++i) {
    s += d[b[i] >> 4];
    s += d[b[i] & 15];
  }
  return s;
}

void put32(std::vector<uint8_t>& b, uint32_t v) {
  for (int k = 0; k < 4; ++k) b.push_back(uint8_t(v >> (8 * k)));
}
void put64(std::vector<uint8_t>& b, uint64_t v) {
  for (int k = 0; k < 8; ++k) b.push_back(uint8_t(v >> (8 * k)));
}
void put64s(std::string& b, uint64_t v) {
  for (int k = 0; k < 8; ++k) b += char(uint8_t(v >> (8 * k)));
}
uint32_t get32(const uint8_t* p) { return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24; }
uint64_t get64(const uint8_t* p) { return uint64_t(get32(p)) | uint64_t(get32(p + 4)) << 32; }

uint64_t round_up(uint64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool is_uuid(const std::string& s) {
  if (s.size() != 36) return false;
  for (size_t i = 0; i < 36; ++i) {
    const char c = s[i];
    if (i == 8 || i == 13 || i == 18 || i == 23) {
      if (c != '-') return false;
    } else if (!std::isxdigit(uint8_t(c))) {
      return false;
    }
  }
  return true;
}

std::string optimizer_json(const CheckpointOptimizer& o) {
  std::string s = std::string("{\"kind\":\"") + (o.adamw ? "AdamW" : "Sgd") + "\",\"learning_rate\":" + json_f64(o.learning_rate);
  if (o.adamw)
    s += ",\"weight_decay\":" + json_f64(o.weight_decay) + ",\"beta1\":" + json_f64(o.beta1) + ",\"beta2\":" +
         json_f64(o.beta2) + ",\"epsilon\":" + json_f64(o.epsilon) + ",\"schedule\":{\"warmup_steps\":" +
         std::to_string(o.warmup_steps) + "}";
  return s + "}";
}

std::string record_json(const CheckpointTensor& t, uint64_t offset, uint64_t length) {
  std::string s = "{\"path\":" + json::quote(t.path);
  if (!t.slot.empty()) s += ",\"slot\":" + json::quote(t.slot);
  s += ",\"dtype\":\"F32\",\"shape\":[";
  for (size_t i = 0; i < t.shape.size(); ++i) s += (i ? "," : "") + std::to_string(t.shape[i]);
  return s + "],\"offset\":" + std::to_string(offset) + ",\"length\":" + std::to_string(length) + "}";
}

[[noreturn]] void refuse(const char* code, const std::string& shown, const std::string& what) {
  throw CheckpointError(code, what + " (" + shown + ")");
}

// Only the named keys, each once (serde's deny_unknown_fields and duplicate-field errors).
void only_keys(const json::Value& v, std::initializer_list<const char*> allowed, const std::string& what) {
  if (v.kind != json::Value::Object) throw std::runtime_error(what + " is not an object");
  std::set<std::string> seen;
  for (auto& [k, x] : v.fields) {
    bool ok = false;
    for (const char* a : allowed) ok = ok || k == a;
    if (!ok) throw std::runtime_error("unknown field `" + k + "` in " + what);
    if (!seen.insert(k).second) throw std::runtime_error("duplicate field `" + k + "` in " + what);
  }
}

CheckpointOptimizer parse_optimizer(const json::Value& v) {
  only_keys(v, {"kind", "learning_rate", "weight_decay", "beta1", "beta2", "epsilon", "schedule", "muon"}, "optimizer");
  CheckpointOptimizer o;
  const std::string& kind = v.at("kind").str();
  if (kind != "Sgd" && kind != "AdamW") throw std::runtime_error("optimizer kind `" + kind + "` is not Sgd or AdamW");
  o.adamw = kind == "AdamW";
  o.learning_rate = v.at("learning_rate").number();
  const char* adam_fields[] = {"weight_decay", "beta1", "beta2", "epsilon", "schedule"};
  int present = 0;
  for (const char* f : adam_fields) present += v.find(f) && v.find(f)->kind != json::Value::Null;
  // OptimizerConfig::is_valid (checkpoint.rs:152-168).
  if (!std::isfinite(o.learning_rate) || (o.adamw ? present != 5 : present != 0) ||
      (v.find("muon") && v.find("muon")->kind != json::Value::Null))
    throw std::runtime_error("the optimizer's fields do not fit its kind");
  if (o.adamw) {
    o.weight_decay = v.at("weight_decay").number();
    o.beta1 = v.at("beta1").number();
    o.beta2 = v.at("beta2").number();
    o.epsilon = v.at("epsilon").number();
    const json::Value& sch = v.at("schedule");
    only_keys(sch, {"warmup_steps"}, "schedule");
    o.warmup_steps = sch.at("warmup_steps").u64();
  }
  return o;
}

struct Record {
  std::string path, slot;
  std::vector<uint64_t> shape;
  uint64_t offset = 0, length = 0;
};

Record parse_record(const json::Value& v) {
  only_keys(v, {"path", "slot", "dtype", "shape", "offset", "length"}, "a record");
  Record r;
  r.path = v.at("path").str();
  if (const json::Value* s = v.find("slot"); s && s->kind != json::Value::Null) r.slot = s->str();
  if (v.at("dtype").str() != "F32") throw std::runtime_error("a dtype other than F32");
  const json::Value& sh = v.at("shape");
  if (sh.kind != json::Value::Array) throw std::runtime_error("a shape that is not a list");
  if (sh.items.size() > kMaxRank) throw std::runtime_error("a shape has more than 8 dimensions");
  for (auto& d : sh.items) r.shape.push_back(d.u64());
  r.offset = v.at("offset").u64();
  r.length = v.at("length").u64();
  return r;
}

}  // namespace

std::string json_f64(double v) {
  if (!std::isfinite(v)) throw IrError("a checkpoint holds no infinite or NaN hyperparameter");
  if (v == 0) return std::signbit(v) ? "-0.0" : "0.0";
  // The shortest digits that read back as v, and the decimal exponent: v = 0.d1d2..dn x 10^kk.
  char buf[64];
  int prec = 1;
  for (; prec <= 17; ++prec) {
    std::snprintf(buf, sizeof buf, "%.*e", prec - 1, v);
    if (std::strtod(buf, nullptr) == v) break;
  }
  std::string text = buf;
  const bool neg = text[0] == '-';
  if (neg) text = text.substr(1);
  const size_t e = text.find('e');
  std::string digits;
  for (size_t i = 0; i < e; ++i)
    if (text[i] != '.') digits += text[i];
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  const int exp10 = std::atoi(text.c_str() + e + 1);
  const int n = int(digits.size()), k = exp10 - (n - 1), kk = n + k;
  std::string out;
  if (k >= 0 && kk <= 16) {
    out = digits + std::string(size_t(k), '0') + ".0";
  } else if (kk > 0 && kk <= 16) {
    out = digits.substr(0, size_t(kk)) + "." + digits.substr(size_t(kk));
  } else if (kk > -5 && kk <= 0) {
    out = "0." + std::string(size_t(-kk), '0') + digits;
  } else {
    out = digits.substr(0, 1);
    if (n > 1) out += "." + digits.substr(1);
    out += "e" + std::to_string(kk - 1);
  }
  return neg ? "-" + out : out;
}

namespace json {
Value real(double v) {
  Value x;
  x.kind = Value::Number;
  x.text = json_f64(v);
  x.num = v;
  return x;
}
}  // namespace json

bool CheckpointOptimizer::operator==(const CheckpointOptimizer& o) const {
  if (adamw != o.adamw || learning_rate != o.learning_rate) return false;
  return !adamw || (weight_decay == o.weight_decay && beta1 == o.beta1 && beta2 == o.beta2 && epsilon == o.epsilon &&
                    warmup_steps == o.warmup_steps);
}

std::string schema_hash(const Program& p) {
  std::string b = "modelspec-schema/1\n";
  for (auto& d : p.params) {
    put64s(b, d.path.size());
    b += d.path;
    b += d.ty.dtype == DType::F32 ? "f32" : "i32";
    put64s(b, uint64_t(d.ty.rank()));
    for (int64_t n : d.ty.shape) {
      b += char(0);
      put64s(b, uint64_t(n));
    }
  }
  uint8_t h[32];
  blake3(b.data(), b.size(), h);
  return hexs(h, 32);
}

CheckpointOptimizer optimizer_of(const TrainingStep& step) {
  CheckpointOptimizer o;
  o.learning_rate = double(step.lr);
  if (step.rule == Rule::AdamW) {
    o.adamw = true;
    o.weight_decay = double(step.adamw.weight_decay);
    o.beta1 = double(step.adamw.beta1);
    o.beta2 = double(step.adamw.beta2);
    o.epsilon = double(step.adamw.eps);
    o.warmup_steps = step.adamw.warmup_steps;
  }
  return o;
}

Checkpoint checkpoint_of(const TrainingStep& step, uint64_t seed, uint64_t updates,
                         const std::vector<std::vector<float>>& values, const std::vector<std::vector<float>>& m,
                         const std::vector<std::vector<float>>& v) {
  const Program& p = step.program;
  if (values.size() != p.params.size()) throw IrError("a checkpoint needs every parameter's value");
  Checkpoint c;
  c.step = updates;
  c.schema_hash = schema_hash(p);
  c.optimizer = optimizer_of(step);
  c.seed = seed;
  auto shape_of = [&](size_t q) {
    std::vector<uint64_t> s;
    for (int64_t n : p.params[q].ty.shape) s.push_back(uint64_t(n));
    return s;
  };
  for (size_t q = 0; q < p.params.size(); ++q) {
    if (int64_t(values[q].size()) != p.params[q].ty.count()) throw IrError("`" + p.params[q].path + "` has the wrong size");
    c.parameters.push_back({p.params[q].path, "", shape_of(q), values[q]});
    if (step.rule == Rule::AdamW && step.moments.count(uint32_t(q))) {
      if (q < m.size() && !m[q].empty()) c.slots.push_back({p.params[q].path, "m", shape_of(q), m[q]});
      if (q < v.size() && !v[q].empty()) c.slots.push_back({p.params[q].path, "v", shape_of(q), v[q]});
    }
  }
  std::sort(c.parameters.begin(), c.parameters.end(), [](auto& a, auto& b) { return a.path < b.path; });
  std::sort(c.slots.begin(), c.slots.end(),
            [](auto& a, auto& b) { return a.path != b.path ? a.path < b.path : a.slot < b.slot; });
  return c;
}

std::vector<uint8_t> encode(const Checkpoint& c) {
  for (auto* list : {&c.parameters, &c.slots})
    for (auto& t : *list)
      if (t.shape.size() > kMaxRank)
        throw CheckpointError("E-CKPT-002", "parameter `" + t.path + "` has more than 8 dimensions");
  // The payload: each tensor at a multiple of 64 from the payload start, zero bytes between.
  std::vector<uint8_t> payload;
  std::vector<std::pair<uint64_t, uint64_t>> rel;
  for (auto* list : {&c.parameters, &c.slots})
    for (auto& t : *list) {
      const uint64_t at = round_up(payload.size());
      payload.resize(size_t(at), 0);
      const uint8_t* raw = reinterpret_cast<const uint8_t*>(t.data.data());
      payload.insert(payload.end(), raw, raw + t.data.size() * 4);  // little-endian host
      rel.push_back({at, uint64_t(t.data.size()) * 4});
    }
  uint8_t ph[32];
  blake3(payload.data(), payload.size(), ph);
  const std::string payload_hash = hexs(ph, 32);
  auto manifest = [&](uint64_t start, const std::string& id) {
    std::string s = "{\"checkpoint_id\":" + json::quote(id) + ",\"file_size\":" + std::to_string(start + payload.size()) +
                    ",\"alignment\":64,\"schema_hash\":" + json::quote(c.schema_hash) + ",\"step\":" +
                    std::to_string(c.step) + ",\"payload_hash\":" + json::quote(payload_hash) +
                    ",\"optimizer\":" + optimizer_json(c.optimizer) + ",\"optimizer_slots\":[";
    size_t i = c.parameters.size();
    for (size_t k = 0; k < c.slots.size(); ++k, ++i)
      s += (k ? "," : "") + record_json(c.slots[k], start + rel[i].first, rel[i].second);
    s += "],\"rng\":{\"algorithm\":\"Philox4x32x10\",\"seed\":" + std::to_string(c.seed) + ",\"counter\":" +
         std::to_string(c.counter) + "},\"parameters\":[";
    for (size_t k = 0; k < c.parameters.size(); ++k)
      s += (k ? "," : "") + record_json(c.parameters[k], start + rel[k].first, rel[k].second);
    return s + "]}";
  };
  // The payload start depends on the manifest's length, which depends on the offsets in it.
  uint64_t start = 0;
  std::string unnamed;
  while (true) {
    unnamed = manifest(start, kNilUuid);
    const uint64_t next = round_up(kHeader + unnamed.size());
    if (next == start) break;
    start = next;
  }
  std::string idb = "modelspec-checkpoint-id/1\n" + unnamed;
  uint8_t idh[32];
  blake3(idb.data(), idb.size(), idh);
  const std::string named = manifest(start, uuid_of(idh));
  std::vector<uint8_t> bytes;
  bytes.insert(bytes.end(), {'M', 'S', 'C', 'K'});
  put32(bytes, kVersion);
  put32(bytes, kEndian);
  put32(bytes, 0);
  put64(bytes, named.size());
  bytes.resize(kHeader, 0);
  bytes.insert(bytes.end(), named.begin(), named.end());
  uint8_t sum[32];
  blake3(bytes.data(), bytes.size(), sum);
  std::memcpy(bytes.data() + 24, sum, 32);
  bytes.resize(size_t(start), 0);
  bytes.insert(bytes.end(), payload.begin(), payload.end());
  return bytes;
}

void write_checkpoint(const std::string& path, const Checkpoint& c) {
  const std::vector<uint8_t> bytes = encode(c);
  const std::string staged = path + ".tmp";
  {
    std::ofstream f(staged, std::ios::binary | std::ios::trunc);
    if (!f) throw IrError("cannot write checkpoint " + path + ": " + std::strerror(errno));
    f.write(reinterpret_cast<const char*>(bytes.data()), std::streamsize(bytes.size()));
    f.flush();
    if (!f) {
      std::remove(staged.c_str());
      throw IrError("cannot write checkpoint " + path + ": a short write");
    }
  }
  if (std::rename(staged.c_str(), path.c_str()) != 0) {
    std::remove(staged.c_str());
    throw IrError("cannot write checkpoint " + path + ": " + std::strerror(errno));
  }
}

Checkpoint read_checkpoint(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) refuse("E-CKPT-001", path, "not a readable checkpoint: the file cannot be read");
  std::ostringstream s;
  s << f.rdbuf();
  const std::string text = s.str();
  return decode_checkpoint(std::vector<uint8_t>(text.begin(), text.end()), path);
}

Checkpoint decode_checkpoint(const std::vector<uint8_t>& bytes, const std::string& shown) {
  const uint64_t size = bytes.size();
  if (size < kHeader)
    refuse("E-CKPT-002", shown, "the file has " + std::to_string(size) + " bytes, fewer than the 56-byte header");
  const uint8_t* h = bytes.data();
  if (std::memcmp(h, "MSCK", 4) != 0) refuse("E-CKPT-001", shown, "not a readable checkpoint: the magic is not MSCK");
  if (get32(h + 4) != kVersion)
    refuse("E-CKPT-001", shown, "not a readable checkpoint: format version " + std::to_string(get32(h + 4)) + " is not 1");
  if (get32(h + 8) != kEndian)
    refuse("E-CKPT-001", shown,
           get32(h + 8) == 0x04030201 ? "not a readable checkpoint: the endian marker is big-endian"
                                      : "not a readable checkpoint: the endian marker is unknown");
  if (get32(h + 12) != 0) refuse("E-CKPT-001", shown, "not a readable checkpoint: the reserved header field is not zero");
  const uint64_t msize = get64(h + 16);
  if (msize == 0 || msize > size - kHeader)
    refuse("E-CKPT-002", shown, "the manifest size " + std::to_string(msize) + " does not fit the file after its header");
  {
    std::vector<uint8_t> signed_bytes(bytes.begin(), bytes.begin() + long(kHeader + msize));
    std::memset(signed_bytes.data() + 24, 0, 32);
    uint8_t sum[32];
    blake3(signed_bytes.data(), signed_bytes.size(), sum);
    if (std::memcmp(sum, h + 24, 32) != 0)
      refuse("E-CKPT-001", shown, "not a readable checkpoint: the checksum differs from the header and manifest");
  }
  const uint64_t manifest_end = kHeader + msize, payload_start = std::min(round_up(manifest_end), size);
  const std::string mtext(bytes.begin() + long(kHeader), bytes.begin() + long(manifest_end));
  Checkpoint c;
  std::vector<Record> params, slots;
  uint64_t file_size = 0, alignment = 0;
  std::string checkpoint_id, payload_hash;
  try {
    json::Value m = json::parse(mtext);
    only_keys(m, {"checkpoint_id", "file_size", "alignment", "schema_hash", "step", "payload_hash", "optimizer",
                  "optimizer_slots", "rng", "parameters"},
              "the manifest");
    checkpoint_id = m.at("checkpoint_id").str();
    file_size = m.at("file_size").u64();
    alignment = m.at("alignment").u64();
    c.schema_hash = m.at("schema_hash").str();
    c.step = m.at("step").u64();
    payload_hash = m.at("payload_hash").str();
    c.optimizer = parse_optimizer(m.at("optimizer"));
    const json::Value& rng = m.at("rng");
    only_keys(rng, {"algorithm", "seed", "counter"}, "rng");
    if (rng.at("algorithm").str() != "Philox4x32x10") throw std::runtime_error("an unknown rng algorithm");
    c.seed = rng.at("seed").u64();
    c.counter = rng.at("counter").u64();
    const json::Value& pl = m.at("parameters");
    const json::Value& sl = m.at("optimizer_slots");
    if (pl.kind != json::Value::Array || sl.kind != json::Value::Array) throw std::runtime_error("records are not lists");
    const uint64_t most = (size + kSlack) / kRecordBytes;
    if (pl.items.size() + sl.items.size() > most)
      refuse("E-CKPT-002", shown,
             "the manifest has " + std::to_string(pl.items.size() + sl.items.size()) + " records, more than the " +
                 std::to_string(most) + " a " + std::to_string(size) + "-byte file can hold");
    for (auto& r : pl.items) params.push_back(parse_record(r));
    for (auto& r : sl.items) slots.push_back(parse_record(r));
  } catch (const CheckpointError&) {
    throw;
  } catch (const std::exception& e) {
    refuse("E-CKPT-001", shown, std::string("not a readable checkpoint: the manifest is not a checkpoint manifest: ") + e.what());
  }
  // The manifest's own invariants (checkpoint.rs:872-921).
  auto bad = [&](const std::string& w) { refuse("E-CKPT-001", shown, "not a readable checkpoint: " + w); };
  if (!is_uuid(checkpoint_id)) bad("checkpoint_id is not a UUID");
  if (!c.optimizer.adamw && !slots.empty()) bad("an SGD checkpoint has optimizer slots");
  if (params.empty()) bad("the manifest has no parameter");
  {
    std::set<std::string> paths;
    for (auto& r : params) {
      if (!r.slot.empty()) bad("parameter `" + r.path + "` has a slot name");
      if (!paths.insert(r.path).second) bad("parameter `" + r.path + "` is recorded twice");
    }
    std::set<std::pair<std::string, std::string>> named;
    for (auto& r : slots) {
      if (r.slot.empty()) bad("an optimizer slot of `" + r.path + "` has no name");
      if (!named.insert({r.path, r.slot}).second) bad("slot `" + r.slot + "` of `" + r.path + "` is recorded twice");
    }
    for (auto* list : {&params, &slots})
      for (auto& r : *list) {
        for (uint64_t d : r.shape)
          if (d == 0) bad("parameter `" + r.path + "` has a zero dimension");
        if (r.length == 0) bad("parameter `" + r.path + "` has length 0");
      }
  }
  auto outside = [&](const std::string& w) { refuse("E-CKPT-002", shown, w); };
  if (file_size != size)
    outside("the manifest's file_size " + std::to_string(file_size) + " is not the file's " + std::to_string(size) + " bytes");
  if (alignment != kAlign) outside("the alignment " + std::to_string(alignment) + " is not 64");
  std::vector<std::tuple<uint64_t, uint64_t, std::string>> extents;
  for (auto* list : {&params, &slots})
    for (auto& r : *list) {
      const std::string at = "parameter `" + r.path + "`: ";
      if (r.offset % kAlign) outside(at + "offset " + std::to_string(r.offset) + " is not a multiple of 64");
      if (r.offset < manifest_end) outside(at + "offset " + std::to_string(r.offset) + " lies inside the header or manifest");
      if (r.length > size || r.offset > size - r.length) outside(at + "the tensor ends past the file");
      unsigned __int128 want = 4;
      for (uint64_t d : r.shape) want *= d;
      if (want != r.length) outside(at + "length " + std::to_string(r.length) + " is not the shape's elements times 4 bytes");
      extents.emplace_back(r.offset, r.offset + r.length, r.path);
    }
  std::sort(extents.begin(), extents.end());
  for (size_t i = 1; i < extents.size(); ++i)
    if (std::get<0>(extents[i]) < std::get<1>(extents[i - 1]))
      outside("parameters `" + std::get<2>(extents[i - 1]) + "` and `" + std::get<2>(extents[i]) + "` overlap");
  uint64_t last = manifest_end;
  for (auto& e : extents) last = std::max(last, std::get<1>(e));
  if (last != size) outside("the file does not end at the end of its last tensor");
  uint64_t cursor = manifest_end;
  for (auto& e : extents) {
    for (uint64_t b = cursor; b < std::get<0>(e); ++b)
      if (bytes[size_t(b)]) outside("byte " + std::to_string(b) + " lies between tensors and is not zero");
    cursor = std::get<1>(e);
  }
  uint8_t ph[32];
  blake3(bytes.data() + payload_start, size_t(size - payload_start), ph);
  if (hexs(ph, 32) != payload_hash) refuse("E-CKPT-004", shown, "the payload hash differs from the payload");
  auto tensor = [&](const Record& r) {
    CheckpointTensor t{r.path, r.slot, r.shape, std::vector<float>(size_t(r.length / 4))};
    std::memcpy(t.data.data(), bytes.data() + r.offset, size_t(r.length));
    return t;
  };
  for (auto& r : params) c.parameters.push_back(tensor(r));
  for (auto& r : slots) c.slots.push_back(tensor(r));
  return c;
}

std::vector<std::vector<float>> parameters_for(const Checkpoint& c, const TrainingStep& step) {
  const Program& p = step.program;
  std::vector<std::pair<std::string, size_t>> ours;
  for (size_t q = 0; q < p.params.size(); ++q) ours.push_back({p.params[q].path, q});
  std::sort(ours.begin(), ours.end());
  std::vector<std::vector<float>> values(p.params.size());
  const std::string lead = "the checkpoint does not match the compiled file: ";
  for (size_t i = 0; i < std::max(ours.size(), c.parameters.size()); ++i) {
    const CheckpointTensor* theirs = i < c.parameters.size() ? &c.parameters[i] : nullptr;
    const std::pair<std::string, size_t>* mine = i < ours.size() ? &ours[i] : nullptr;
    if (!theirs || !mine || theirs->path != mine->first)
      throw CheckpointError("E-CKPT-003", lead + "a parameter path differs (checkpoint " +
                                             (theirs ? "`" + theirs->path + "`" : std::string("none")) +
                                             ", compiled file " + (mine ? "`" + mine->first + "`" : std::string("none")) + ")");
    const ParamDecl& d = p.params[mine->second];
    if (d.ty.dtype != DType::F32)
      throw CheckpointError("E-CKPT-003", lead + "parameter `" + d.path + "` has dtype f32 in the checkpoint and i32 in the compiled file");
    std::vector<uint64_t> shape;
    for (int64_t n : d.ty.shape) shape.push_back(uint64_t(n));
    if (shape != theirs->shape)
      throw CheckpointError("E-CKPT-003", lead + "parameter `" + d.path + "` has another shape");
    values[mine->second] = theirs->data;
  }
  if (schema_hash(p) != c.schema_hash) throw CheckpointError("E-CKPT-003", lead + "the schema hash differs");
  return values;
}

ResumeState resume_into(const Checkpoint& c, const TrainingStep& step) {
  ResumeState r;
  r.step = c.step;
  r.values = parameters_for(c, step);
  if (optimizer_of(step) != c.optimizer)
    throw CheckpointError("E-CKPT-003", "the checkpoint does not match the compiled file: the optimizer differs");
  const Program& p = step.program;
  r.m.assign(p.params.size(), {});
  r.v.assign(p.params.size(), {});
  if (step.rule != Rule::AdamW) return r;
  std::map<std::pair<std::string, std::string>, const CheckpointTensor*> slot;
  for (auto& t : c.slots) slot[{t.path, t.slot}] = &t;
  for (auto& [param, mo] : step.moments) {
    const ParamDecl& d = p.params[param];
    for (const char* which : {"m", "v"}) {
      auto it = slot.find({d.path, which});
      std::vector<float>& dst = which[0] == 'm' ? r.m[param] : r.v[param];
      if (it == slot.end()) {
        if (c.step != 0)
          throw CheckpointError("E-CKPT-003", "the checkpoint does not match the compiled file: AdamW moment `" +
                                                  std::string(which) + "` of `" + d.path + "` is missing after step " +
                                                  std::to_string(c.step));
        dst.assign(size_t(d.ty.count()), 0.0f);
      } else {
        std::vector<uint64_t> shape;
        for (int64_t n : d.ty.shape) shape.push_back(uint64_t(n));
        if (it->second->shape != shape)
          throw CheckpointError("E-CKPT-003", "the checkpoint does not match the compiled file: moment `" +
                                                  std::string(which) + "` of `" + d.path + "` has another shape");
        dst = it->second->data;
      }
    }
  }
  return r;
}

}  // namespace msx
