// The binding a maintainer adds to audio.cpp's src/framework/runtime/
// host_ops.cpp (the body INTEGRATION.md shows), compiled here against the
// reference's own declaration of engine::runtime::VectorQuantizer
// (include/engine/framework/runtime/host_ops.h:87-96, from the reference
// tree at build time; nothing of it is copied).  Test infrastructure: it
// replaces the reference's host loop (src/framework/runtime/host_ops.cpp:
// 236-273) with the MI355X library and is linked into ref_adapter_parity.
#include "engine/framework/runtime/host_ops.h"

#include "aq_mi355x.hpp"

namespace engine::runtime {

FloatHostTensor VectorQuantizer::compute(const std::vector<float> &input, const std::vector<float> &codebook,
                                         int64_t batch, int64_t steps, int64_t dim, int64_t codebook_size) const {
    thread_local aq::Context ctx(0);   // one context per calling thread
    const auto r = aq::engine::runtime::VectorQuantizer(ctx).compute(input, codebook, batch, steps, dim, codebook_size);
    return FloatHostTensor{r.values, r.shape};
}

}  // namespace engine::runtime
