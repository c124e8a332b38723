// The device side of a staged upload. The host copies small uploads into a slot of the context's
// pinned staging ring (coherent host memory mapped into the device's address space), and one
// kernel copies every upload of the call from there to its destination. One launch then replaces
// one host-to-device copy per upload, which for the tables of a verify step costs most of the
// time (each copy is queued as a transfer of its own).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "kernels.hpp"

namespace kyro {
namespace {

__global__ __launch_bounds__(256) void upload_scatter_kernel(UploadArgs a) {
    const int u = blockIdx.y;
    const uint64_t* src = reinterpret_cast<const uint64_t*>(a.src + a.off[u]);
    uint64_t* dst = a.dst[u];
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.words[u]; i += (int64_t)gridDim.x * 256)
        dst[i] = src[i];
}

}  // namespace

hipError_t launch_upload_scatter(const UploadArgs& a, hipStream_t stream) {
    if (a.n <= 0) return hipSuccess;
    int64_t most = 0;
    for (int u = 0; u < a.n; ++u) most = std::max(most, a.words[u]);
    const unsigned gx = (unsigned)std::max<int64_t>(1, std::min<int64_t>((most + 255) / 256, 64));
    upload_scatter_kernel<<<dim3(gx, (unsigned)a.n), 256, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace kyro
