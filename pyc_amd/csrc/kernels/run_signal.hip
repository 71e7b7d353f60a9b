// run_signal.hip — a host-visible completion word for the backend's runs.
//
// A synchronous run (pyc_run_model returns once its outputs exist) normally
// ends in hipStreamSynchronize, whose notification path (completion signal,
// then the runtime's wait) takes several microseconds after the last kernel
// ends. Instead, the backend enqueues this one-lane kernel behind the run's
// work on the same stream: stream order starts it only after that work has
// completed (and its writes were released at the kernel boundary), and it
// stores the run's sequence number into pinned, host-coherent memory with a
// system-scope release. The host spins on that word with an acquire load.
// The reference waits with cudaStreamSynchronize
// (reference src/compiler/runtime/cuda_backend.c:1845-1849, 2214-2218); this is the
// MI355X replacement for that wait, not a change of what the run guarantees.
#include "common.hpp"

namespace pyc {

__global__ void __launch_bounds__(kWave) run_signal_kernel(uint32_t* __restrict__ word, uint32_t seq) {
    if (threadIdx.x == 0) __hip_atomic_store(word, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace pyc

// Enqueues the completion store of `seq` into `host_word` (pinned memory
// allocated with hipHostMallocCoherent) on `stream`. 0, or -2 on a HIP error.
extern "C" int pyc_hip_run_signal_enqueue(uint32_t* host_word, uint32_t seq, void* stream) {
    if (!host_word) return -2;
    hipLaunchKernelGGL(pyc::run_signal_kernel, dim3(1), dim3(pyc::kWave), 0, (hipStream_t)stream, host_word, seq);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
