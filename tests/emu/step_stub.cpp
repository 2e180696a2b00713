// Host entry points of the persistent decode step for the CPU emulation
// build.  That kernel (its LDS ring fed by direct-to-LDS loads and its
// inter-workgroup polling) is not emulated: the stub reports that no
// persistent grid fits, so contexts take the one-kernel-per-op decode path.
// TEST INFRASTRUCTURE ONLY.
#include "launch.h"

namespace sq {

bool decode_step_fits(int, int, int, int, int) { return false; }
size_t decode_stream_stride(int, int, int, int, int, int, int, int) { return 0; }
size_t exchange_words(int, int, int, int, int, int) { return 0; }
int launch_build_stream(hipStream_t, int, const StepArgs&, int, void*) {
    return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step is not emulated");
}
int launch_decode_step(hipStream_t, int, const StepArgs&, int, int) {
    return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step is not emulated");
}
int decode_step_max_grid(int, int* grid) {
    *grid = 0;
    return 0;
}

}  // namespace sq
