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
// Where the run's last kernel can do it, that kernel stores the word itself
// (run_signal_claim, run_signal_arrive) and this kernel is not launched.
// The reference waits with cudaStreamSynchronize
// (reference src/compiler/runtime/cuda_backend.c:1845-1849, 2214-2218); this is the
// MI355X replacement for that wait, not a change of what the run guarantees.
#include "common.hpp"

namespace pyc {

__global__ void __launch_bounds__(kWave) run_signal_kernel(uint32_t* __restrict__ word, uint32_t seq) {
    if (threadIdx.x == 0) __hip_atomic_store(word, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Armed signal of the calling thread (the run path arms, launches its last
// kernel and takes the result on one thread; per thread, so that a GEMM
// another thread dispatches meanwhile cannot claim it).
struct PendingSignal {
    RunSignal sig{nullptr, nullptr, 0};
    bool armed = false, taken = false;
};
thread_local PendingSignal g_pending;

bool run_signal_claim(RunSignal* out) {
    if (!g_pending.armed) return false;
    *out = g_pending.sig;
    g_pending.armed = false;
    g_pending.taken = true;
    return true;
}

}  // namespace pyc

// Arms the completion store of `seq` for the next kernel launched on this
// thread that can store it itself (`dev_count`: 9 x 256 bytes of device
// memory, zero).
extern "C" void pyc_hip_run_signal_arm(uint32_t* host_word, uint32_t* dev_count, uint32_t seq) {
    pyc::g_pending.sig = pyc::RunSignal{host_word, dev_count, seq};
    pyc::g_pending.armed = host_word != nullptr && dev_count != nullptr;
    pyc::g_pending.taken = false;
}

// 1 when a launch since the arm claimed the signal; disarms either way.
extern "C" int pyc_hip_run_signal_taken(void) {
    const int t = pyc::g_pending.taken ? 1 : 0;
    pyc::g_pending.armed = false;
    pyc::g_pending.taken = false;
    return t;
}

// Enqueues the completion store of `seq` into `host_word` (pinned memory
// allocated with hipHostMallocCoherent) on `stream`. 0, or -2 on a HIP error.
extern "C" int pyc_hip_run_signal_enqueue(uint32_t* host_word, uint32_t seq, void* stream) {
    if (!host_word) return -2;
    hipLaunchKernelGGL(pyc::run_signal_kernel, dim3(1), dim3(pyc::kWave), 0, (hipStream_t)stream, host_word, seq);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
