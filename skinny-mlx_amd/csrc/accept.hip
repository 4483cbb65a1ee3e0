// Greedy acceptance of the verify step, on the device.
//
// Reference behaviour: skinny_mlx/spec.py:137-147 — pred = argmax over each verify row
// (mx.argmax: the first maximal index), n = the longest prefix with draft[i] == pred[i],
// emitted tokens draft[:n] + [pred[n]], cache rolled back to keep = n + 1 of fed = K + 1.
#include "common.h"

namespace {

constexpr int kThreads = 1024;

// (value, index) with first-index ties: larger value wins, equal values keep the lower index.
__device__ __forceinline__ void better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// One workgroup per row; bf16 logits with row stride ld.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const uint16_t* __restrict__ logits, int V, int ld,
                                                          int32_t* __restrict__ pred) {
  const uint16_t* row = logits + (size_t)blockIdx.x * ld;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < V; i += kThreads) better(bv, bi, bf16_bits_to_f32(row[i]), i);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) better(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
  __shared__ float sv[kThreads / 64];
  __shared__ int si[kThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w) better(bv, bi, sv[w], si[w]);
    pred[blockIdx.x] = bi == 0x7fffffff ? 0 : bi;
  }
}

// out[0] = n (accepted drafts), out[1] = bonus token pred[n], out[2] = keep = n + 1.
__global__ void accept_kernel(const int32_t* __restrict__ pred, const int32_t* __restrict__ draft, int k,
                              int32_t* __restrict__ out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int n = 0;
  while (n < k && draft[n] == pred[n]) ++n;
  out[0] = n;
  out[1] = pred[n];
  out[2] = n + 1;
}

}  // namespace

extern "C" int skinny_argmax_rows_bf16(const uint16_t* logits, int rows, int V, int ld, int32_t* pred, void* stream) {
  SKINNY_CHECK_ARG(logits && pred, "argmax: null pointer");
  SKINNY_CHECK_ARG(rows >= 1 && V >= 1 && ld >= V, "argmax: bad shape rows=%d V=%d ld=%d", rows, V, ld);
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, logits, V, ld, pred);
  return skinny_check_launch("argmax");
}

extern "C" int skinny_accept(const int32_t* pred, const int32_t* draft, int k, int32_t* out, void* stream) {
  SKINNY_CHECK_ARG(pred && out && (k == 0 || draft), "accept: null pointer");
  SKINNY_CHECK_ARG(k >= 0, "accept: k=%d must be >= 0", k);
  hipLaunchKernelGGL(accept_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, pred, draft, k, out);
  return skinny_check_launch("accept");
}
