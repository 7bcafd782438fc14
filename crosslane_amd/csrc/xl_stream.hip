// Streaming single-launch layer (the kernel: xl_stream.hpp): the IQ2_XXS
// gate/up + IQ2_XS down instance, and the choice between the instances.
#include "xl_stream.hpp"

namespace xl::dev {

hipError_t launch_stream(const Layer3Args& args, int gu_types, int dn_types, int cus, hipStream_t s, hipEvent_t stop) {
    if (gu_types == 1 && dn_types == 2 && args.slab) return launch_stream_shapes<1, 2>(args, cus, s, stop);
    if (gu_types == 4 && dn_types == 4 && args.slab) {
        const hipError_t e = launch_stream_iq1(args, cus, s, stop);
        if (e != hipErrorNotSupported) return e;
    }
    if ((gu_types & ~7) || (dn_types & ~7) || !gu_types || !dn_types) return hipErrorNotSupported;
    return launch_stream_mix(args, cus, s, stop);
}

}  // namespace xl::dev
