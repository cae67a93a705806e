// A compiled artifact of format version 1 with the `Hip` backend: artifact.json and one gfx950
// code object per kernel module under kernels/.
//
// Restates the on-disk form of crates/modelspec-core/src/artifact.rs:1-35, 210-520 for this
// backend: the manifest keys of format 1 (format_version, artifact_id, backend, artifact_hash,
// source_hash, ir_hash, fast_math, deterministic, compiler_version, schema_hash, parameters,
// data, kernels, plan, forward_plan, buffers, loss_view, prediction_view) in serde_json's pretty
// form; `artifact_hash` is BLAKE3 over the manifest with artifact_hash and artifact_id empty,
// then each module's bytes in module-id order; `artifact_id` its first 16 bytes as a version-8
// UUID. Where the Vulkan artifact holds SPIR-V modules and a kernel-IR plan, a Hip artifact holds
// the gfx950 code objects this library was built with and the plan this library made from the
// printed training step, which the manifest carries (`step_ir`, `forward_ir`, the boundary the
// runtime plans from); `ir_hash` is BLAKE3 of `step_ir`, as the reference hashes print_step.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "ir.h"

namespace msx {

// A refused artifact: `code` E-ARTIFACT-001 (no readable manifest of a known version and of the
// Hip backend), 002 (a module, the artifact hash or id differs from what the manifest records,
// or the modules are not this library's), 003 (an invariant: a module that is not a gfx950 code
// object, an ir_hash, schema or parameter that does not match the step, a plan too long), 004 (a
// module file missing, not regular, longer than its entry, or a stray file in kernels/), 005 (a
// device other than the artifact's target).
struct ArtifactError : IrError {
  ArtifactError(const std::string& code, const std::string& what) : IrError(code + ": " + what), code(code) {}
  std::string code;
};

struct ArtifactLaunch {
  std::string what;
  double flop = 0, bytes = 0;
};

// What a Hip artifact is written from.
struct ArtifactSource {
  std::string source_text;  // the text the step was compiled from (source_hash)
  std::string step_ir, forward_ir;  // print.rs text of the training step and forward program
  uint32_t prediction_output = 1;   // index of the prediction among the forward outputs
  std::vector<int64_t> param_offsets;  // per ParamId, floats into the parameter arena
  int64_t param_floats = 0;
  std::vector<ArtifactLaunch> plan, forward_plan;
  std::string code_objects;     // the directory of this library's *.hsaco
  std::string target = "gfx950";
  std::string compiler_version;
};

struct HipArtifact {
  std::string artifact_id, artifact_hash, source_hash, ir_hash, schema_hash, compiler_version, target;
  std::string step_ir, forward_ir;
  uint32_t prediction_output = 1;
  uint64_t plan_launches = 0, forward_launches = 0;
  std::vector<std::string> module_hashes;  // blake3 of each code object, in module-id order
};

// Writes the artifact to `dir` (created if missing; an earlier artifact.json and kernels/ in it
// are replaced); returns the artifact hash.
std::string write_artifact(const std::string& dir, const ArtifactSource& src);

// Reads and validates `dir` in the reference's order (manifest, module files, module hashes,
// artifact hash and id, invariants); with `code_objects` non-empty, also refuses (E-ARTIFACT-002)
// modules other than the code objects in that directory, the ones this library runs.
HipArtifact read_artifact(const std::string& dir, const std::string& code_objects);

// The BLAKE3 hex digest of each *.hsaco in `dir`, by file name order.
std::vector<std::pair<std::string, std::string>> code_object_hashes(const std::string& dir);

}  // namespace msx
