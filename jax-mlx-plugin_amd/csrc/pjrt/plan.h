// Static launch plan of one compiled module.
//
// Shapes are static, so everything the reference decides per call (op
// dispatch through an if-chain, tier selection, mx::compile tracing —
// reference src/jax_mlx_pjrt.cpp:3040-3195, 8920-9434) is decided once here:
// every value gets a place (caller parameter, uploaded constant, output
// buffer, or an offset in one reusable arena sized by liveness), and Execute
// replays a flat list of kernel launches on one HIP stream.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "ir.h"
#include "mfx_kernels.h"

namespace mfxp {

// Where a value's bytes live at execution time.
struct Loc {
  enum Kind : uint8_t { kNone, kParam, kConst, kArena, kOutput } kind = kNone;
  int index = 0;       // param / const / output index
  int64_t offset = 0;  // bytes (arena offset, or extra offset for views)
};

struct ExecBuffers {
  std::vector<void*> params;
  std::vector<void*> outputs;
  void* arena = nullptr;
  hipStream_t stream = nullptr;
};

struct Step {
  std::string kind;   // "elementwise", "gemm", "reduce", "layer_norm", ... (for tracing)
  std::string label;  // op / kernel detail
  double flops = 0;
  double bytes = 0;
  std::vector<int> reads, writes;  // value ids the step reads / writes (aliases resolved), for inspection
  // Resolves pointers and launches; returns MFX_OK or an error code.
  std::function<int(const ExecBuffers&, std::string&)> run;
};

class Plan {
 public:
  // Builds the plan of `f` (already rewritten); throws ParseError on
  // unsupported ops.
  static std::unique_ptr<Plan> build(const Function& f);
  ~Plan();

  const std::vector<Type>& param_types() const { return params_; }
  const std::vector<Type>& result_types() const { return results_; }
  size_t arena_bytes() const { return arena_bytes_; }
  const std::vector<Step>& steps() const { return steps_; }
  double total_flops() const;
  std::string summary_json() const;

  // Uploads constants to the current device (once).
  int prepare(std::string& err);
  // Enqueues every step on b.stream.  `outputs` must hold result buffers.
  int run(ExecBuffers& b, std::string& err);

  // Filled by the planner.
  std::vector<Type> params_, results_;
  std::vector<std::shared_ptr<Literal>> const_host_;
  std::vector<void*> const_dev_;
  size_t arena_bytes_ = 0;
  void* arena_ = nullptr;
  std::vector<Step> steps_;
  std::mutex mu_;
  bool prepared_ = false;

  // Device pointer of a location (valid inside run()).
  void* ptr(const Loc& l, const ExecBuffers& b) const;
};

int mfx_dtype(DType t);  // DType -> MFX_* code (-1 if none)

}  // namespace mfxp
