// The no-allocation workspace: one fixed device array per GPU that the
// allocation-free entry points (wpcg_linear_gemm_noalloc) carve their
// workspace from, so that a call makes no hipMalloc/hipFree. The array is
// part of the code object: every GPU the library runs on holds its own copy,
// at its own address, until the process ends.
//
// In host code the name `scratch` is a host-side stand-in, not a device
// address. Its device address on a GPU comes from hipGetSymbolAddress, called
// once per device with that device current (scratch_setup, run by
// wpcg_ctx_create); only that address is ever passed to kernels or copies.
#include <hip/hip_runtime.h>

#include <mutex>
#include <unordered_map>

#include "wpcg_internal.hpp"

static __device__ __align__(256) unsigned char scratch[WPCG_NOALLOC_SCRATCH_BYTES];

namespace wpcg {
namespace {

std::mutex g_scratch_mu;
std::unordered_map<int, void*> g_scratch_ptr;  // device -> address of `scratch` on it

__global__ __launch_bounds__(256) void k_fill_u32(uint32_t* __restrict__ p, int n, uint32_t v)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace

int scratch_setup(int device)
{
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (g_scratch_ptr.count(device)) return WPCG_OK;
    int cur = -1;
    WPCG_HIP(hipGetDevice(&cur));
    if (cur != device) return fail(WPCG_E_DEVICE, "scratch set-up: device " + std::to_string(device) + " is not current");
    void* p = nullptr;
    WPCG_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(WPCG_E_DEVICE, "scratch set-up: no device address for the workspace array");
    g_scratch_ptr[device] = p;
    return WPCG_OK;
}

void* scratch_ptr(int device)
{
    std::lock_guard<std::mutex> g(g_scratch_mu);
    auto it = g_scratch_ptr.find(device);
    return it == g_scratch_ptr.end() ? nullptr : it->second;
}

hipError_t launch_fill_u32(uint32_t* p, int n, uint32_t v, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

}  // namespace wpcg
