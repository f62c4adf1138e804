// Device scratch for the entry points that allocate nothing
// (svl_bidirectional_attention_noalloc): a file-scope device array, one copy
// per GPU, holding what the allocating entry point puts in per-call device
// allocations: the attention work-item list, the per-token position and row
// length arrays of the generic kernel, and the non-finite flag.
//
// Host code must never pass `scratch` itself to a kernel or a copy: in host
// code that name is a host-side stand-in, not a device address. Its device
// address is looked up once per device with hipGetSymbolAddress (with that
// device current) and kept in g_scratch_ptr; every use goes through it.
#include <mutex>

#include "svl_internal.hpp"

namespace svl {

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 256;
std::mutex g_scratch_mu;
void *g_scratch_ptr[MAX_DEVICES] = {};
}  // namespace

hipError_t noalloc_scratch(int device, void **out) {
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        int current = 0;
        hipError_t e = hipGetDevice(&current);
        if (e != hipSuccess) return e;
        if (current != device && (e = hipSetDevice(device)) != hipSuccess) return e;
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (current != device) (void)hipSetDevice(current);
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

// Fills the scratch for one attention call over a single row of `seq` keys:
// work item i of KV head g = i / per_head covers query vectors
// (i % per_head) * bv .. + bv - 1 (the order the allocating entry point
// builds on the host), pos[t] = t, rowlen[t] = seq, and the flag is cleared
// (a kernel rather than a memset, so the call can sit in a captured graph).
__global__ void noalloc_attn_setup_kernel(unsigned char *base, int seq, int per_head, int bv,
                                          int n_tiles) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n_tiles) {
        AttnTile *tiles = (AttnTile *)(base + NOALLOC_TILES_OFF);
        const int g = i / per_head;
        tiles[i] = AttnTile{0, seq, g, (i - g * per_head) * bv};
    }
    if (i < seq) {
        ((int32_t *)(base + NOALLOC_POS_OFF))[i] = i;
        ((int32_t *)(base + NOALLOC_LEN_OFF))[i] = seq;
    }
    if (i == 0) *(int *)(base + NOALLOC_FLAG_OFF) = 0;
}

hipError_t launch_noalloc_attn_setup(void *base, int seq, int per_head, int bv, int n_tiles,
                                     hipStream_t s) {
    const int n = std::max(std::max(seq, n_tiles), 1);
    hipLaunchKernelGGL(noalloc_attn_setup_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       s, (unsigned char *)base, seq, per_head, bv, n_tiles);
    return hipGetLastError();
}

}  // namespace svl
