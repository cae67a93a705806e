// The Hip artifact of artifact.h.
#include "artifact.h"

#include <dirent.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <sstream>

#include "checkpoint.h"
#include "json.h"
#include "packed.h"
#include "rng.h"

namespace msx {
namespace {

const char* kManifest = "artifact.json";
const char* kKernels = "kernels";
constexpr uint64_t kMaxManifest = uint64_t(64) << 20;
constexpr size_t kMaxPlan = 4096;  // MAX_PLAN_STEPS, core/src/artifact.rs:277

std::string join(const std::string& a, const std::string& b) { return a.empty() || a.back() == '/' ? a + b : a + "/" + b; }

std::string hex(const uint8_t* b, size_t n) {
  static const char* d = "0123456789abcdef";
  std::string s;
  for (size_t i = 0; i < n; ++i) {
    s += d[b[i] >> 4];
    s += d[b[i] & 15];
  }
  return s;
}

std::string blake3_hex(const std::string& bytes) {
  uint8_t h[32];
  blake3(bytes.data(), bytes.size(), h);
  return hex(h, 32);
}

bool read_file(const std::string& path, std::string& out, uint64_t limit) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream s;
  s << f.rdbuf();
  out = s.str();
  return out.size() <= limit;
}

void write_file(const std::string& path, const std::string& bytes) {
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) throw IrError("cannot write " + path + ": " + std::strerror(errno));
  f.write(bytes.data(), std::streamsize(bytes.size()));
  if (!f) throw IrError("cannot write " + path + ": a short write");
}

std::vector<std::string> list_dir(const std::string& dir) {
  std::vector<std::string> out;
  if (DIR* d = opendir(dir.c_str())) {
    while (dirent* e = readdir(d)) {
      std::string n = e->d_name;
      if (n != "." && n != "..") out.push_back(n);
    }
    closedir(d);
  }
  std::sort(out.begin(), out.end());
  return out;
}

void remove_tree(const std::string& path) {
  struct stat st;
  if (lstat(path.c_str(), &st) != 0) return;
  if (S_ISDIR(st.st_mode)) {
    for (auto& n : list_dir(path)) remove_tree(join(path, n));
    rmdir(path.c_str());
  } else {
    unlink(path.c_str());
  }
}

// A gfx950 code object: a 64-bit little-endian ELF of machine EM_AMDGPU (224).
bool is_amdgpu_elf(const std::string& b) {
  return b.size() >= 64 && std::memcmp(b.data(), "\x7f" "ELF", 4) == 0 && b[4] == 2 && b[5] == 1 &&
         uint8_t(b[18]) == 0xE0 && uint8_t(b[19]) == 0;
}

json::Value view(uint64_t buffer, uint64_t count, uint64_t offset_bytes) {
  json::Value v = json::object();
  json::put(v, "buffer", json::uint(buffer));
  json::put(v, "dtype", json::str("f32"));
  json::put(v, "element_count", json::uint(count));
  json::put(v, "offset", json::uint(offset_bytes));
  json::put(v, "size_bytes", json::uint(count * 4));
  json::put(v, "alignment", json::uint(4));
  return v;
}

json::Value shape_json(const Type& t) {
  json::Value a = json::array();
  for (int64_t n : t.shape) json::push(a, json::uint(uint64_t(n)));
  return a;
}

json::Value plan_json(const std::vector<ArtifactLaunch>& plan) {
  json::Value a = json::array();
  for (size_t i = 0; i < plan.size(); ++i) {
    json::Value s = json::object();
    json::put(s, "step", json::uint(i));
    json::put(s, "launch", json::str(plan[i].what));
    json::put(s, "flop", json::real(plan[i].flop));
    json::put(s, "bytes", json::real(plan[i].bytes));
    json::push(a, std::move(s));
  }
  return a;
}

// BLAKE3 over the manifest with artifact_hash and artifact_id empty, then the modules in id order
// (core/src/artifact.rs:1541-1560).
std::string artifact_hash(json::Value manifest, const std::vector<std::pair<std::string, std::string>>& modules) {
  for (auto& [k, v] : manifest.fields)
    if (k == "artifact_hash" || k == "artifact_id") v = json::str("");
  std::string bytes = json::dump_pretty(manifest) + "\n";
  for (auto& [id, b] : modules) bytes += b;
  return blake3_hex(bytes);
}

std::string uuid_of_hex(const std::string& h) {
  uint8_t b[32];
  for (int i = 0; i < 32; ++i) b[i] = uint8_t(std::stoi(h.substr(size_t(2 * i), 2), nullptr, 16));
  return uuid_of(b);
}

}  // namespace

std::vector<std::pair<std::string, std::string>> code_object_hashes(const std::string& dir) {
  std::vector<std::pair<std::string, std::string>> out;
  for (auto& n : list_dir(dir)) {
    if (n.size() < 6 || n.substr(n.size() - 6) != ".hsaco") continue;
    std::string b;
    if (!read_file(join(dir, n), b, UINT64_MAX)) throw IrError("cannot read code object " + join(dir, n));
    out.push_back({n, blake3_hex(b)});
  }
  return out;
}

std::string write_artifact(const std::string& dir, const ArtifactSource& src) {
  const TrainingStep step = parse_step(src.step_ir);
  const Program forward = parse_program(src.forward_ir);
  // The code objects, by module id (a UUID of their hash).
  std::vector<std::tuple<std::string, std::string, std::string>> modules;  // id, name, bytes
  for (auto& n : list_dir(src.code_objects)) {
    if (n.size() < 6 || n.substr(n.size() - 6) != ".hsaco") continue;
    std::string b;
    if (!read_file(join(src.code_objects, n), b, UINT64_MAX) || !is_amdgpu_elf(b))
      throw IrError("code object " + join(src.code_objects, n) + " is not a readable gfx950 ELF");
    modules.emplace_back(uuid_of_hex(blake3_hex(b)), n.substr(0, n.size() - 6), b);
  }
  if (modules.empty()) throw IrError("no code objects in " + src.code_objects);
  std::sort(modules.begin(), modules.end());

  json::Value m = json::object();
  json::put(m, "format_version", json::uint(1));
  json::put(m, "artifact_id", json::str(""));
  json::put(m, "backend", json::str("Hip"));
  json::put(m, "artifact_hash", json::str(""));
  json::put(m, "source_hash", json::str(blake3_hex(src.source_text)));
  json::put(m, "ir_hash", json::str(blake3_hex(src.step_ir)));
  json::put(m, "fast_math", json::boolean(false));
  json::put(m, "deterministic", json::boolean(true));
  json::put(m, "compiler_version", json::str(src.compiler_version));
  json::put(m, "schema_hash", json::str(schema_hash(step.program)));
  // Buffers: the four parameter-state arenas (values, gradients, m, v share offsets), then the
  // input block of the step and of the forward program, then the loss log.
  enum { kParams, kGrads, kM, kV, kStepInputs, kForwardInputs, kLossLog };
  json::Value params = json::array();
  for (size_t q = 0; q < step.program.params.size(); ++q) {
    const ParamDecl& d = step.program.params[q];
    json::Value p = json::object();
    json::put(p, "param", json::uint(q));
    json::put(p, "path", json::str(d.path));
    json::put(p, "canonical_parameter_id", json::uint(canonical_id(d.path)));
    json::put(p, "dtype", json::str("f32"));
    json::put(p, "shape", shape_json(d.ty));
    json::Value views = json::array();
    const uint64_t off = q < src.param_offsets.size() ? uint64_t(src.param_offsets[q]) * 4 : 0;
    json::push(views, view(kParams, uint64_t(d.ty.count()), off));
    json::put(p, "views", std::move(views));
    json::push(params, std::move(p));
  }
  json::put(m, "parameters", std::move(params));
  // Data: the forward program's inputs; the ones a loss reads as its target or weights are targets.
  std::set<uint32_t> targets;
  for (auto& n : forward.nodes) {
    if (n.op == Op::CrossEntropy) targets.insert({n.operands[1], n.operands[2]});
    if (n.op == Op::Mse) targets.insert(n.operands[1]);
  }
  json::Value data = json::array();
  uint64_t at = 0;
  for (auto& n : forward.nodes)
    if (n.op == Op::Input) {
      json::Value d = json::object();
      json::put(d, "name", json::str(n.name));
      json::put(d, "role", json::str(targets.count(n.id) ? "Target" : "Input"));
      json::put(d, "dtype", json::str(n.ty.dtype == DType::F32 ? "f32" : "i32"));
      json::put(d, "shape", shape_json(n.ty));
      json::put(d, "view", view(kForwardInputs, uint64_t(n.ty.count()), at));
      at += (uint64_t(n.ty.count()) * 4 + 255) / 256 * 256;
      json::push(data, std::move(d));
    }
  json::put(m, "data", std::move(data));
  json::Value kernels = json::array();
  for (auto& [id, name, bytes] : modules) {
    json::Value k = json::object();
    json::put(k, "kernel_module_id", json::str(id));
    json::put(k, "entry_point", json::str(name));
    json::Value key = json::object();
    json::put(key, "ir_hash", json::str(blake3_hex(src.step_ir)));
    json::put(key, "shapes", json::array());
    json::put(key, "dtype", json::str("f32"));
    json::put(key, "fast_math", json::boolean(false));
    json::put(key, "deterministic", json::boolean(true));
    json::put(key, "vendor_id", json::uint(0x1002));
    json::put(key, "device_id", json::uint(0));
    json::put(key, "driver_version", json::uint(0));
    json::Value caps = json::array();
    json::push(caps, json::str(src.target));
    json::put(key, "capabilities", std::move(caps));
    json::put(k, "cache_key", std::move(key));
    json::put(k, "byte_length", json::uint(bytes.size()));
    json::put(k, "blake3", json::str(blake3_hex(bytes)));
    json::put(k, "kind", json::str("code_object"));
    json::put(k, "op", json::str(name));
    json::put(k, "dtype", json::str("f32"));
    json::put(k, "operands", json::array());
    json::push(kernels, std::move(k));
  }
  json::put(m, "kernels", std::move(kernels));
  if (src.plan.size() > kMaxPlan || src.forward_plan.size() > kMaxPlan) throw IrError("a plan of more than 4096 launches");
  json::put(m, "plan", plan_json(src.plan));
  json::put(m, "forward_plan", plan_json(src.forward_plan));
  json::Value buffers = json::array();
  const char* names[] = {"parameters", "gradients", "adamw_m", "adamw_v", "step_inputs", "forward_inputs", "loss_log"};
  for (int b = 0; b < 7; ++b) {
    json::Value x = json::object();
    json::put(x, "buffer", json::uint(uint64_t(b)));
    json::put(x, "name", json::str(names[b]));
    json::put(x, "size_bytes", json::uint(b <= kV ? uint64_t(src.param_floats) * 4 : b == kForwardInputs ? at : 0));
    json::push(buffers, std::move(x));
  }
  json::put(m, "buffers", std::move(buffers));
  json::put(m, "loss_view", view(kLossLog, 1, 0));
  json::put(m, "prediction_view", [&] {
    json::Value v = json::object();
    json::put(v, "output", json::uint(src.prediction_output));
    return v;
  }());
  json::put(m, "target", json::str(src.target));
  json::put(m, "step_ir", json::str(src.step_ir));
  json::put(m, "forward_ir", json::str(src.forward_ir));

  std::vector<std::pair<std::string, std::string>> by_id;
  for (auto& [id, name, bytes] : modules) by_id.push_back({id, bytes});
  const std::string hash = artifact_hash(m, by_id);
  for (auto& [k, v] : m.fields) {
    if (k == "artifact_hash") v = json::str(hash);
    if (k == "artifact_id") v = json::str(uuid_of_hex(hash));
  }
  // Replace an earlier artifact: modules first, the manifest last.
  if (mkdir(dir.c_str(), 0755) != 0 && errno != EEXIST) throw IrError("cannot create " + dir + ": " + std::strerror(errno));
  remove_tree(join(dir, kManifest));
  remove_tree(join(dir, kKernels));
  if (mkdir(join(dir, kKernels).c_str(), 0755) != 0) throw IrError("cannot create " + join(dir, kKernels));
  for (auto& [id, name, bytes] : modules) write_file(join(join(dir, kKernels), id + ".hsaco"), bytes);
  write_file(join(dir, kManifest), json::dump_pretty(m) + "\n");
  return hash;
}

HipArtifact read_artifact(const std::string& dir, const std::string& code_objects) {
  const std::string mpath = join(dir, kManifest);
  auto refuse = [&](const char* code, const std::string& what) -> ArtifactError {
    return ArtifactError(code, what + " (" + dir + ")");
  };
  struct stat st;
  if (lstat(mpath.c_str(), &st) != 0 || !S_ISREG(st.st_mode)) throw refuse("E-ARTIFACT-001", "artifact.json is missing or not a regular file");
  if (uint64_t(st.st_size) > kMaxManifest) throw refuse("E-ARTIFACT-001", "artifact.json is larger than 64 MiB");
  std::string text;
  if (!read_file(mpath, text, kMaxManifest)) throw refuse("E-ARTIFACT-001", "artifact.json cannot be read");
  json::Value m;
  try {
    m = json::parse(text);
    if (m.at("format_version").u64() != 1) throw refuse("E-ARTIFACT-001", "format_version is not 1");
    if (m.at("backend").str() != "Hip")
      throw refuse("E-ARTIFACT-001", "an artifact of the " + m.at("backend").str() + " backend; this library runs Hip");
  } catch (const ArtifactError&) {
    throw;
  } catch (const std::exception& e) {
    throw refuse("E-ARTIFACT-001", std::string("artifact.json is not a manifest: ") + e.what());
  }
  HipArtifact a;
  std::vector<std::tuple<std::string, uint64_t, std::string>> entries;  // id, byte_length, blake3
  try {
    a.artifact_id = m.at("artifact_id").str();
    a.artifact_hash = m.at("artifact_hash").str();
    a.source_hash = m.at("source_hash").str();
    a.ir_hash = m.at("ir_hash").str();
    a.schema_hash = m.at("schema_hash").str();
    a.compiler_version = m.at("compiler_version").str();
    a.target = m.at("target").str();
    a.step_ir = m.at("step_ir").str();
    a.forward_ir = m.at("forward_ir").str();
    a.prediction_output = uint32_t(m.at("prediction_view").at("output").u64());
    const json::Value& plan = m.at("plan");
    const json::Value& fplan = m.at("forward_plan");
    if (plan.items.size() > kMaxPlan || fplan.items.size() > kMaxPlan)
      throw refuse("E-ARTIFACT-003", "a plan of more than 4096 steps");
    a.plan_launches = plan.items.size();
    a.forward_launches = fplan.items.size();
    for (auto& k : m.at("kernels").items)
      entries.emplace_back(k.at("kernel_module_id").str(), k.at("byte_length").u64(), k.at("blake3").str());
  } catch (const ArtifactError&) {
    throw;
  } catch (const std::exception& e) {
    throw refuse("E-ARTIFACT-001", std::string("artifact.json is not a manifest: ") + e.what());
  }
  // Module files: each named one regular and no longer than its entry, and nothing else.
  const std::string kdir = join(dir, kKernels);
  std::set<std::string> named;
  for (auto& [id, len, h] : entries) {
    const std::string path = join(kdir, id + ".hsaco");
    if (lstat(path.c_str(), &st) != 0 || !S_ISREG(st.st_mode))
      throw refuse("E-ARTIFACT-004", "kernel module " + path + " is missing or not a regular file");
    if (uint64_t(st.st_size) > len) throw refuse("E-ARTIFACT-004", "kernel module " + path + " is longer than its manifest entry");
    named.insert(id + ".hsaco");
  }
  for (auto& n : list_dir(kdir))
    if (!named.count(n)) throw refuse("E-ARTIFACT-004", "kernels/ holds " + n + ", which no kernel of the manifest names");
  std::vector<std::pair<std::string, std::string>> modules;
  for (auto& [id, len, h] : entries) {
    std::string b;
    const std::string path = join(kdir, id + ".hsaco");
    if (!read_file(path, b, len)) throw refuse("E-ARTIFACT-004", "kernel module " + path + " cannot be read");
    if (blake3_hex(b) != h) throw refuse("E-ARTIFACT-002", "kernel module " + path + " differs from the hash its manifest entry records");
    modules.push_back({id, b});
  }
  std::sort(modules.begin(), modules.end());
  const std::string hash = artifact_hash(m, modules);
  if (hash != a.artifact_hash) throw refuse("E-ARTIFACT-002", "the artifact differs from the artifact_hash its manifest records");
  if (uuid_of_hex(hash) != a.artifact_id) throw refuse("E-ARTIFACT-002", "the artifact_id is not the one its artifact_hash gives");
  // Invariants.
  for (auto& [id, b] : modules)
    if (!is_amdgpu_elf(b)) throw refuse("E-ARTIFACT-003", "the module " + id + " is not an AMDGPU code object");
  if (blake3_hex(a.step_ir) != a.ir_hash) throw refuse("E-ARTIFACT-003", "ir_hash is not the hash of step_ir");
  TrainingStep step;
  try {
    step = parse_step(a.step_ir);
    (void)parse_program(a.forward_ir);
  } catch (const std::exception& e) {
    throw refuse("E-ARTIFACT-003", std::string("step_ir or forward_ir does not parse: ") + e.what());
  }
  if (schema_hash(step.program) != a.schema_hash) throw refuse("E-ARTIFACT-003", "schema_hash is not the step's");
  const json::Value& params = m.at("parameters");
  if (params.items.size() != step.program.params.size()) throw refuse("E-ARTIFACT-003", "the parameters are not the step's");
  for (size_t q = 0; q < params.items.size(); ++q) {
    const json::Value& p = params.items[q];
    const ParamDecl& d = step.program.params[q];
    std::vector<uint64_t> shape;
    for (auto& x : p.at("shape").items) shape.push_back(x.u64());
    std::vector<uint64_t> want;
    for (int64_t n : d.ty.shape) want.push_back(uint64_t(n));
    if (p.at("param").u64() != q || p.at("path").str() != d.path || p.at("canonical_parameter_id").u64() != canonical_id(d.path) ||
        shape != want)
      throw refuse("E-ARTIFACT-003", "parameter " + std::to_string(q) + " is not the step's `" + d.path + "`");
  }
  for (auto& [id, b] : modules) a.module_hashes.push_back(blake3_hex(b));
  if (!code_objects.empty()) {
    std::vector<std::string> ours;
    for (auto& [n, h] : code_object_hashes(code_objects)) ours.push_back(h);
    std::vector<std::string> theirs = a.module_hashes;
    std::sort(ours.begin(), ours.end());
    std::sort(theirs.begin(), theirs.end());
    if (ours != theirs)
      throw refuse("E-ARTIFACT-002", "the artifact's code objects are not the ones this library was built with");
  }
  return a;
}

}  // namespace msx
