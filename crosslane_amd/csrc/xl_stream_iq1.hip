// Streaming single-launch layer (the kernel: xl_stream.hpp), IQ1_M-only instance.
#include "xl_stream.hpp"

namespace xl::dev {

hipError_t launch_stream_iq1(const Layer3Args& args, int cus, hipStream_t s, hipEvent_t stop) {
    return launch_stream_shapes<4, 4>(args, cus, s, stop);
}

}  // namespace xl::dev
