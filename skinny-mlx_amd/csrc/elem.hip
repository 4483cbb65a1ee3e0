// Elementwise pieces of the decoder: SwiGLU activation, embedding gather, and the W4 g64
// dequantisation (to fp32) used by the unpatched (reference-semantics) linear path.
#include "common.h"

namespace {

// act[t, i] = silu(gu[t, i]) * gu[t, F + i]   (gate and up halves of the fused projection)
__global__ void silu_mul_kernel(const uint16_t* __restrict__ gu, int ldg, uint16_t* __restrict__ act, int F) {
  const int t = blockIdx.y;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < F; i += gridDim.x * blockDim.x) {
    const float g = bf16_bits_to_f32(gu[(size_t)t * ldg + i]);
    const float u = bf16_bits_to_f32(gu[(size_t)t * ldg + F + i]);
    act[(size_t)t * F + i] = silu_mul_bf16(g, u);
  }
}

// out[t, :] = table[ids[t], :]; ids out of range raise no fault (row clamped) — the host
// validates ids before launch.
__global__ void embed_kernel(const int32_t* __restrict__ ids, const uint16_t* __restrict__ table, int V, int H,
                             uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  int id = ids[t];
  id = id < 0 ? 0 : (id >= V ? V - 1 : id);
  const uint16_t* src = table + (size_t)id * H;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x) out[(size_t)t * H + i] = src[i];
}

// w[n, k] = q[n, k] * s[n, k/64] + b[n, k/64] in fp32 (MLX packs, element i at bits 4i); q*s is
// exact in fp32, so each weight carries one rounding, like an fp32 dequantise-and-multiply.
__global__ void dequant_kernel(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ sc,
                               const uint16_t* __restrict__ bi, float* __restrict__ out, int N, int K) {
  const size_t words = (size_t)N * (K / 8);
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < words; i += (size_t)gridDim.x * blockDim.x) {
    const size_t n = i / (K / 8);
    const int kw = (int)(i % (K / 8));
    const size_t g = n * (K / 64) + kw / 8;
    const float s = bf16_bits_to_f32(sc[g]), b = bf16_bits_to_f32(bi[g]);
    const uint32_t w = wq[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) out[i * 8 + e] = fmaf((float)((w >> (4 * e)) & 0xFu), s, b);
  }
}

int grid_for(size_t work, int threads) {
  const size_t b = (work + threads - 1) / threads;
  return (int)(b < 65536 ? (b ? b : 1) : 65536);
}

}  // namespace

extern "C" int skinny_silu_mul_bf16(const uint16_t* gate_up, int ld, uint16_t* act, int tokens, int F, void* stream) {
  SKINNY_CHECK_ARG(gate_up && act, "silu_mul: null pointer");
  SKINNY_CHECK_ARG(tokens >= 1 && tokens <= 65535 && F >= 1 && ld >= 2 * F, "silu_mul: bad shape");
  const int gx = grid_for((size_t)F, 256) < 64 ? grid_for((size_t)F, 256) : 64;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(gx, tokens), dim3(256), 0, (hipStream_t)stream, gate_up, ld, act, F);
  return skinny_check_launch("silu_mul");
}

extern "C" int skinny_embed_bf16(const int32_t* ids, int tokens, const uint16_t* table, int V, int H, uint16_t* out,
                                 void* stream) {
  SKINNY_CHECK_ARG(ids && table && out, "embed: null pointer");
  SKINNY_CHECK_ARG(tokens >= 1 && tokens <= 65535 && V >= 1 && H >= 1, "embed: bad shape");
  const int gx = grid_for((size_t)H, 256) < 16 ? grid_for((size_t)H, 256) : 16;
  hipLaunchKernelGGL(embed_kernel, dim3(gx, tokens), dim3(256), 0, (hipStream_t)stream, ids, table, V, H, out);
  return skinny_check_launch("embed");
}

extern "C" int skinny_w4g64_dequant(const uint32_t* w_mlx, const uint16_t* scales, const uint16_t* biases,
                                    float* out, int N, int K, void* stream) {
  SKINNY_CHECK_ARG(w_mlx && scales && biases && out, "dequant: null pointer");
  SKINNY_CHECK_ARG(N >= 1 && K >= 64 && K % 64 == 0, "dequant: bad shape N=%d K=%d", N, K);
  hipLaunchKernelGGL(dequant_kernel, dim3(grid_for((size_t)N * (K / 8), 256)), dim3(256), 0, (hipStream_t)stream,
                     w_mlx, scales, biases, out, N, K);
  return skinny_check_launch("dequant");
}
