// Calibration for the decode GEMVs' roofline: how fast this chip streams a buffer from memory when a kernel does
// nothing else. Measurement equipment for bench.py (liblfm2q_calib.so), not part of the product interface.
//
// Each thread reads `per_lane` 16-byte chunks of the buffer -- chunk (b U + u) 256 + t for workgroup b, u < U, thread
// t -- through a buffer resource whose range is the buffer's length, so a chunk past the end reads zeros and no
// address outside the buffer is touched whatever the grid. The loads of a thread are all issued before any result
// is used (U loads in flight per lane). The XOR of everything read is compared with a value the data cannot produce
// in practice and written only then, so the loads cannot be removed and the kernel writes (almost) nothing.
// aux selects the cache policy of the loads: 0 default (cached: lines allocate in L2 and the memory-side cache),
// 2 non-temporal (streamed once), which is how the GEMVs read their weights.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int THREADS = 256;
constexpr int MAX_U = 16;

template <int U, int AUX>
__global__ __launch_bounds__(THREADS) void stream_read_kernel(const void *__restrict__ src, uint32_t bytes,
                                                              int32_t *__restrict__ out) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(src), (short)0, (int)bytes, 0x00020000);
    v4i v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t chunk = ((uint32_t)blockIdx.x * U + u) * THREADS + threadIdx.x;
        v[u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(chunk * 16u), 0, AUX));
    }
    int x = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    if (x == 0x5a17c0de) out[0] = x;
}

template <int AUX>
int launch(const void *src, uint32_t bytes, int32_t *out, int per_lane, hipStream_t st) {
    const uint32_t per_block = (uint32_t)THREADS * 16u * (uint32_t)per_lane;
    const dim3 grid((bytes + per_block - 1) / per_block);
    switch (per_lane) {
        case 1: stream_read_kernel<1, AUX><<<grid, THREADS, 0, st>>>(src, bytes, out); break;
        case 2: stream_read_kernel<2, AUX><<<grid, THREADS, 0, st>>>(src, bytes, out); break;
        case 4: stream_read_kernel<4, AUX><<<grid, THREADS, 0, st>>>(src, bytes, out); break;
        case 8: stream_read_kernel<8, AUX><<<grid, THREADS, 0, st>>>(src, bytes, out); break;
        default: stream_read_kernel<MAX_U, AUX><<<grid, THREADS, 0, st>>>(src, bytes, out); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace

// Read `bytes` of `src` (16-byte aligned; 16 <= bytes < 2^31, a multiple of 16) once. per_lane: 1, 2, 4, 8 or 16
// loads in flight per lane; aux: 0 (cached) or 2 (non-temporal); out: one int32 of device memory. Returns 0, -1
// for bad arguments, -2 for a launch error.
extern "C" int lfm2q_calib_stream_read(const void *src, size_t bytes, int32_t *out, int per_lane, int aux,
                                       hipStream_t stream) {
    if (!src || !out || ((uintptr_t)src & 15) || bytes < 16 || bytes % 16 || bytes >= 0x80000000ull) return -1;
    if (per_lane != 1 && per_lane != 2 && per_lane != 4 && per_lane != 8 && per_lane != 16) return -1;
    if (aux == 0) return launch<0>(src, (uint32_t)bytes, out, per_lane, stream);
    if (aux == 2) return launch<2>(src, (uint32_t)bytes, out, per_lane, stream);
    return -1;
}
