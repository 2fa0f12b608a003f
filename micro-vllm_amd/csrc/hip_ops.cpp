// hip_ops.cpp -- metal_ops-shaped C++ front end over the HIP C ABI.
#include "hip_ops.hpp"

#include "../../include/mvllm_hip.h"

#include <cstdlib>

namespace mvllm {
namespace hip_ops {

bool init() {
    const char *dev = std::getenv("MVLLM_HIP_DEVICE");
    return mvllm_hip_init(dev ? std::atoi(dev) : 0) == 1;
}

void shutdown() { mvllm_hip_shutdown(); }

bool available() { return mvllm_hip_available() == 1; }

const char *backend_name() { return mvllm_hip_name(); }

bool moe_block(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
               const void *const *u, const void *const *d, const float *const *gs,
               const float *const *us, const float *const *ds, const float *xg, const int *xoff,
               const int *nr, const int *rows, const float *rw, float *out, int S, Act act,
               float act_a, float act_b) {
    return mvllm_hip_moe_block(nb, D, Iinter, fmt, qgs, g, u, d, gs, us, ds, xg, xoff, nr, rows,
                               rw, out, S, static_cast<int>(act), act_a, act_b) == 1;
}

bool moe_block_dev(int nb, int D, int Iinter, int fmt, const void *const *g,
                   const void *const *u, const void *const *d, const float *const *gs,
                   const float *const *us, const float *const *ds, const float *xg_dev,
                   const int *xoff, const int *nr, const int *rows, const float *rw,
                   float *out_dev, int S, Act act, float act_a, float act_b, void *stream) {
    return mvllm_hip_moe_block_dev(nb, D, Iinter, fmt, 0, g, u, d, gs, us, ds, xg_dev, xoff, nr,
                                   rows, rw, out_dev, S, static_cast<int>(act), act_a, act_b,
                                   stream) == 1;
}

}  // namespace hip_ops
}  // namespace mvllm
