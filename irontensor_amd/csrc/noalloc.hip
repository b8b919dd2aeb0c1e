// Device-resident workspace for the entry point that allocates nothing,
// it_flash_attention_backward_noalloc: the per-row values its row pass writes and its dQ + dK/dV
// kernel reads (rowsum(dO * O), and for BF16 the row's LSE; 4 bytes each per query row) live in `scratch`, a static device array of
// IT_NOALLOC_SCRATCH_BYTES. Every GPU the library runs on holds its own copy, at its own address,
// until the process ends. In host code `scratch` names a host-side stand-in, not device memory, so
// its device address is looked up once per device (it_init, with the device current) and only that
// address is handed to kernels.
#include <mutex>

#include "internal.hpp"

namespace {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[IT_NOALLOC_SCRATCH_BYTES / sizeof(float)];

std::mutex g_mu;
void *g_scratch_ptr[kMaxDevices] = {};

}  // namespace

namespace it {

it_status noalloc_init(int device) {
    if (device < 0 || device >= kMaxDevices) return IT_OK;  // the no-allocation entry reports it
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch_ptr[device]) return IT_OK;
    void *ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return fail_hip(err, "hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(IT_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[device] = ptr;
    return IT_OK;
}

void *noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    return g_scratch_ptr[device];
}

}  // namespace it
