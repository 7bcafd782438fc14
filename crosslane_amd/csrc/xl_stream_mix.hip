// Streaming single-launch layer (the kernel: xl_stream.hpp), any mix of IQ2_XXS,
// IQ2_XS and IQ1_M matrices: each pick's matrices from the layer's slab or its
// descriptor, the decoder chosen per slot by the matrix's type.
#include "xl_stream.hpp"

namespace xl::dev {

hipError_t launch_stream_mix(const Layer3Args& args, int cus, hipStream_t s, hipEvent_t stop) {
    return launch_stream_shapes<7, 7>(args, cus, s, stop);
}

}  // namespace xl::dev
