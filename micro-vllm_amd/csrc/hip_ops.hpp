// hip_ops.hpp -- C++ host mirror of the reference's device-ops interface for the
// routed-expert path, backed by the HIP C ABI (include/mvllm_hip.h).
//
// Same names, argument meaning and return convention as mvllm::metal_ops
// (src/gpu/metal_ops.hpp:15-18, 41-44, 99-108), so an engine call site such as
// glm_expert_try_metal (src/model/glm53.cpp:135-153) switches backend by changing
// the namespace.  false = "use the host kernel".
#pragma once

namespace mvllm {
namespace hip_ops {

// init() selects HIP device $MVLLM_HIP_DEVICE (default 0).
bool init();
void shutdown();
bool available();
const char *backend_name();  // "hip"

enum class Act : int { Silu = 0, ClampSwiGLU = 1, Situ = 2 };

// Batched routed-expert block; every pointer is host memory (see metal_ops::moe_block).
bool moe_block(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
               const void *const *u, const void *const *d, const float *const *gs,
               const float *const *us, const float *const *ds, const float *xg, const int *xoff,
               const int *nr, const int *rows, const float *rw, float *out, int S,
               Act act = Act::Silu, float act_a = 0.f, float act_b = 0.f);

// Same block on device-resident weights / activations / output, enqueued on `stream`.
bool moe_block_dev(int nb, int D, int Iinter, int fmt, const void *const *g,
                   const void *const *u, const void *const *d, const float *const *gs,
                   const float *const *us, const float *const *ds, const float *xg_dev,
                   const int *xoff, const int *nr, const int *rows, const float *rw,
                   float *out_dev, int S, Act act, float act_a, float act_b, void *stream);

}  // namespace hip_ops
}  // namespace mvllm
