// Streaming-read ceiling: the achievable HBM read bandwidth that the skinny qmm is
// compared against beside the 8 TB/s spec (the MI355X counterpart of the reference's
// bench/hw_roofline.py:3-11, which reduces a large buffer to time a streaming read).
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4_t* __restrict__ src, size_t n16,
                                                          float* __restrict__ out) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  // four independent 16-byte loads in flight per iteration
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4_t a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const u32x4_t a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] ^= red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = __uint_as_float(red[0] & 0x007fffffu);  // finite, never NaN
}

// Each workgroup reads its own contiguous chunk of the buffer, kL 16-byte loads in flight per
// thread. Loads past the chunk's end re-read its last piece (no branch between the loads of one
// round, so all of them issue together).
template <int kL>
__global__ __launch_bounds__(256) void stream_read_chunk_kernel(const u32x4_t* __restrict__ src, size_t n16,
                                                                size_t per_wg16, float* __restrict__ out) {
  const size_t b0 = (size_t)blockIdx.x * per_wg16;
  const size_t b1 = b0 + per_wg16 < n16 ? b0 + per_wg16 : n16;
  uint32_t acc = 0;
  if (b0 < b1) {
    for (size_t i = b0 + threadIdx.x; i < b1; i += (size_t)256 * kL) {
      u32x4_t v[kL];
#pragma unroll
      for (int l = 0; l < kL; ++l) {
        const size_t j = i + (size_t)l * 256;
        v[l] = src[j < b1 ? j : b1 - 1];
      }
#pragma unroll
      for (int l = 0; l < kL; ++l) acc ^= v[l].x ^ v[l].y ^ v[l].z ^ v[l].w;
    }
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] ^= red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = __uint_as_float(red[0] & 0x007fffffu);  // finite, never NaN
}

}  // namespace

extern "C" int skinny_stream_read(const void* buf, size_t bytes, float* out, int grid, void* stream) {
  SKINNY_CHECK_ARG(buf && out, "stream_read: null pointer");
  SKINNY_CHECK_ARG(bytes >= 16 && bytes % 16 == 0, "stream_read: bytes=%zu must be a positive multiple of 16", bytes);
  SKINNY_CHECK_ARG(skinny_aligned(buf, 16), "stream_read: buffer must be 16-byte aligned");
  SKINNY_CHECK_ARG(grid >= 1 && grid <= 1 << 20, "stream_read: grid=%d out of range", grid);
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const u32x4_t*>(buf), bytes / 16, out);
  return skinny_check_launch("stream_read");
}

extern "C" int skinny_stream_read_chunked(const void* buf, size_t bytes, float* out, int grid, int loads, void* stream) {
  SKINNY_CHECK_ARG(buf && out, "stream_read_chunked: null pointer");
  SKINNY_CHECK_ARG(bytes >= 16 && bytes % 16 == 0, "stream_read_chunked: bytes=%zu must be a positive multiple of 16",
                   bytes);
  SKINNY_CHECK_ARG(skinny_aligned(buf, 16), "stream_read_chunked: buffer must be 16-byte aligned");
  SKINNY_CHECK_ARG(grid >= 1 && grid <= 1 << 20, "stream_read_chunked: grid=%d out of range", grid);
  SKINNY_CHECK_ARG(loads == 4 || loads == 8 || loads == 16, "stream_read_chunked: loads=%d (4, 8 or 16)", loads);
  const size_t n16 = bytes / 16;
  const size_t per = (n16 + grid - 1) / grid;
  auto kern = loads == 4 ? stream_read_chunk_kernel<4> : (loads == 8 ? stream_read_chunk_kernel<8> : stream_read_chunk_kernel<16>);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, (hipStream_t)stream, reinterpret_cast<const u32x4_t*>(buf), n16,
                     per, out);
  return skinny_check_launch("stream_read_chunked");
}
