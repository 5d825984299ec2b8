// Streaming device copy: the measured HBM ceiling that bench.py reports the bandwidth-bound kernels'
// fractions against (read + write bytes per second), and the known-size reference for the FETCH_SIZE /
// WRITE_SIZE counter runs.  Each lane moves 4 x 16 bytes per iteration (all four loads issued before
// the stores), workgroups stride over the buffer; an unaligned head or tail is copied bytewise.
#include "tesm_hip_internal.h"

namespace tesm {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void stream_copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                          int64_t n16) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256 * 4;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 * 4 + threadIdx.x;
  for (; i + 3 * 256 < n16; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    const u32x4 b = __builtin_nontemporal_load(src + i + 256);
    const u32x4 c = __builtin_nontemporal_load(src + i + 512);
    const u32x4 d = __builtin_nontemporal_load(src + i + 768);
    __builtin_nontemporal_store(a, dst + i);
    __builtin_nontemporal_store(b, dst + i + 256);
    __builtin_nontemporal_store(c, dst + i + 512);
    __builtin_nontemporal_store(d, dst + i + 768);
  }
  for (int k = 0; k < 4; ++k, i += 256)
    if (i < n16) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void byte_copy_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                        int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

int launch_stream_copy(void* dst, const void* src, int64_t bytes, hipStream_t st) {
  TESM_REQUIRE(bytes >= 0 && (bytes == 0 || (dst && src)), kErrInvalidArg, "stream copy: bad arguments");
  if (bytes == 0) return kOk;
  int64_t n16 = 0;
  if (aligned(dst, 16) && aligned(src, 16)) {
    n16 = bytes / 16;
    if (n16 > 0) {
      const int64_t per_wg = 256 * 4;
      const int64_t want = (n16 + per_wg - 1) / per_wg;
      const unsigned grid = static_cast<unsigned>(std::min<int64_t>(want, 256 * 16));
      stream_copy_kernel<<<grid, 256, 0, TESM_LOGGED(st, stream_copy_kernel)>>>(
          static_cast<u32x4*>(dst), static_cast<const u32x4*>(src), n16);
    }
  }
  const int64_t done = n16 * 16, rest = bytes - done;
  if (rest > 0) {
    const unsigned grid = static_cast<unsigned>((rest + 255) / 256);
    byte_copy_kernel<<<grid, 256, 0, TESM_LOGGED(st, byte_copy_kernel)>>>(
        static_cast<uint8_t*>(dst) + done, static_cast<const uint8_t*>(src) + done, rest);
  }
  return check_launch("stream copy");
}

}  // namespace tesm
