// Static device scratch of the allocation-free product entry point
// (qimm_qmatmul_noalloc): the split-K partial sums and arrival counters that
// qimm_qmatmul keeps in the context's growable scratch live here instead, in a
// file-scope device array that every device holds from the library's load
// until the process ends. Host code never passes the array's name to a kernel:
// on the host that name is only a stand-in. Its device address is looked up
// once per device (hipGetSymbolAddress, with that device current) and that
// pointer is what the kernels get.
#include <mutex>

#include "kernels.h"

namespace qimm {

static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void *g_ptr[MAX_DEVICES] = {};

__global__ void zero_words(uint32_t *p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace

hipError_t noalloc_scratch_setup(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    if (g_ptr[device]) return hipSuccess;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    // the arrival counters at the front start at zero; every call leaves them
    // zero again. A fill kernel (no memset node), waited for here so that a
    // call on any stream sees zeros.
    const int64_t words = (int64_t)(STREAM_COUNTER_BYTES / 4);
    zero_words<<<dim3((unsigned)((words + 255) / 256)), dim3(256), 0, nullptr>>>((uint32_t *)p, words);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return e;
    g_ptr[device] = p;
    return hipSuccess;
}

void *noalloc_scratch(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    return (device >= 0 && device < MAX_DEVICES) ? g_ptr[device] : nullptr;
}

}  // namespace qimm
