// Row normalisations of the decoder (fp32 arithmetic, bf16 in/out).
//
// Each row is reduced by one workgroup with a fixed-shape tree, so a row's result never
// depends on how many rows share the launch (the property speculative verify relies on to
// match single-token decoding bit for bit).
#include <array>
#include <utility>

#include "common.h"

namespace {

constexpr int kThreads = 512;  // one workgroup per row; 512 issue the row's loads faster than 256 (0.3 us per launch)

// The sum of squares of a row, in the order the norm-in matmuls reproduce: per thread a fused
// multiply-add chain over its chunks' values in order (chunk c, then c + kThreads), wave_sum of the
// 64 lanes, then the kThreads / 64 wave sums in order starting from 0.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) t += red[w];
  return t;
}

// out = rmsnorm(x (+ res)) * w ; sum_out = x + res rounded to bf16 (the residual stream).
// Single pass: each thread loads its 16-byte chunks (8 values) of the row, the residual and the
// weight into registers at once, so the row costs one memory round trip; the sum of squares
// is reduced in a fixed order (chunk, DPP row sums, rows, waves). sum_out may alias x: a
// thread rewrites only the chunks it has already read.
//
// The residual may instead come as `splits` fp32 slices of a split-K matmul (parts: slice s at
// s * pstride floats, row stride ldp): it is their sum in split order, rounded to bf16, which is
// what the unsplit matmul's output would be up to the order of its fp32 additions.
constexpr int kRowChunks = 2;  // 16-byte chunks per thread: H <= 8 * 2 * 512 = 8192
constexpr int kMaxSplits = 4;

// The row length and the split count come first among the arguments: every load's bounds depend
// on them, and the leading argument dwords arrive preloaded in SGPRs; eps fills the padding after
// ldp, so it is preloaded too, and sum_out (stored mid-kernel) comes before out (stored last).
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(int H, int splits, const uint16_t* x,
                                                           const uint16_t* __restrict__ res,
                                                           const float* __restrict__ parts, size_t pstride, int ldp,
                                                           float eps, const uint16_t* __restrict__ w,
                                                           uint16_t* sum_out, uint16_t* __restrict__ out) {
  __shared__ float red[kThreads / 64];
  const size_t row = blockIdx.x;
  const int nchunk = H >> 3;
  const u32x4_t* xr = reinterpret_cast<const u32x4_t*>(x + row * H);
  const u32x4_t* rr = res ? reinterpret_cast<const u32x4_t*>(res + row * H) : nullptr;
  const u32x4_t* wr = reinterpret_cast<const u32x4_t*>(w);
  u32x4_t xv[kRowChunks], rv[kRowChunks], wv[kRowChunks];
  f32x4_t pv[kRowChunks][kMaxSplits][2];
#pragma unroll
  for (int i = 0; i < kRowChunks; ++i) {  // row, residual and weight chunks all in one round trip
    const int c = threadIdx.x + i * kThreads;
    if (c < nchunk) {
      xv[i] = xr[c];
      if (rr) rv[i] = rr[c];
      wv[i] = wr[c];
      if (parts) {
#pragma unroll
        for (int sp = 0; sp < kMaxSplits; ++sp)
          if (sp < splits) {
            const f32x4_t* src = reinterpret_cast<const f32x4_t*>(parts + sp * pstride + row * ldp + (size_t)c * 8);
            pv[i][sp][0] = src[0];
            pv[i][sp][1] = src[1];
          }
      }
    }
  }
  // The output pointers lie past the preloaded argument dwords: fetch them now, under the row's loads,
  // rather than where they are first used.
  asm volatile("" ::"s"(sum_out), "s"(out));
  if (parts) {  // the residual chunks from the slices
#pragma unroll
    for (int i = 0; i < kRowChunks; ++i) {
      const int c = threadIdx.x + i * kThreads;
      if (c >= nchunk) continue;
      float r[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = pv[i][0][e >> 2][e & 3];
#pragma unroll
      for (int sp = 1; sp < kMaxSplits; ++sp)
        if (sp < splits) {
#pragma unroll
          for (int e = 0; e < 8; ++e) r[e] += pv[i][sp][e >> 2][e & 3];
        }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        rv[i][q] = (uint32_t)f32_to_bf16_bits(r[2 * q]) | ((uint32_t)f32_to_bf16_bits(r[2 * q + 1]) << 16);
    }
    rr = xr;  // non-null: the residual is present (rv holds it)
  }
  float v[kRowChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kRowChunks; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c >= nchunk) continue;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t word = xv[i][e >> 1];
      float f = bf16_bits_to_f32((e & 1) ? (word >> 16) : (word & 0xffffu));
      if (rr) {
        const uint32_t rw = rv[i][e >> 1];
        f = bf16_bits_to_f32(f32_to_bf16_bits(f + bf16_bits_to_f32((e & 1) ? (rw >> 16) : (rw & 0xffffu))));
      }
      v[i][e] = f;
      ss = fmaf(f, f, ss);
    }
    if (sum_out) {
      u32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = (uint32_t)f32_to_bf16_bits(v[i][2 * q]) | ((uint32_t)f32_to_bf16_bits(v[i][2 * q + 1]) << 16);
      reinterpret_cast<u32x4_t*>(sum_out + row * H)[c] = o;
    }
  }
  const float inv = rsqrtf(block_sum(ss, red) / (float)H + eps);
  u32x4_t* orow = reinterpret_cast<u32x4_t*>(out + row * H);
#pragma unroll
  for (int i = 0; i < kRowChunks; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c >= nchunk) continue;
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float w0 = bf16_bits_to_f32(wv[i][q] & 0xffffu), w1 = bf16_bits_to_f32(wv[i][q] >> 16);
      o[q] = (uint32_t)f32_to_bf16_bits(v[i][2 * q] * inv * w0) |
             ((uint32_t)f32_to_bf16_bits(v[i][2 * q + 1] * inv * w1) << 16);
    }
    orow[c] = o;
  }
}

// The MTP head's input rows: workgroup b < T normalises the embedding row of ids[b] (clamped to
// [0, V), as the embedding lookup does) with w_e into out[b, 0:H], workgroup T + b the hidden row b
// with w_h into out[b, H:2H]: the concatenation the head's fc projection reads. Each row is
// rmsnorm_kernel's residual-free arithmetic (same chunks, same reduction order), so it is bitwise
// that kernel's row.
__global__ __launch_bounds__(kThreads) void mtp_input_kernel(int H, int T, const int32_t* __restrict__ ids,
                                                             const uint16_t* __restrict__ table, int V,
                                                             const uint16_t* __restrict__ hidden, int ldh,
                                                             const uint16_t* __restrict__ w_e,
                                                             const uint16_t* __restrict__ w_h, float eps,
                                                             uint16_t* __restrict__ out) {
  __shared__ float red[kThreads / 64];
  const int b = blockIdx.x;
  const bool emb = b < T;
  const int t = emb ? b : b - T;
  const uint16_t* src;
  if (emb) {
    int id = ids[t];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    src = table + (size_t)id * H;
  } else {
    src = hidden + (size_t)t * ldh;
  }
  const u32x4_t* xr = reinterpret_cast<const u32x4_t*>(src);
  const u32x4_t* wr = reinterpret_cast<const u32x4_t*>(emb ? w_e : w_h);
  const int nchunk = H >> 3;
  u32x4_t xv[kRowChunks], wv[kRowChunks];
#pragma unroll
  for (int i = 0; i < kRowChunks; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c < nchunk) {
      xv[i] = xr[c];
      wv[i] = wr[c];
    }
  }
  float v[kRowChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kRowChunks; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c >= nchunk) continue;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t word = xv[i][e >> 1];
      const float f = bf16_bits_to_f32((e & 1) ? (word >> 16) : (word & 0xffffu));
      v[i][e] = f;
      ss = fmaf(f, f, ss);
    }
  }
  const float inv = rsqrtf(block_sum(ss, red) / (float)H + eps);
  u32x4_t* orow = reinterpret_cast<u32x4_t*>(out + (size_t)t * 2 * H + (emb ? 0 : H));
#pragma unroll
  for (int i = 0; i < kRowChunks; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c >= nchunk) continue;
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float w0 = bf16_bits_to_f32(wv[i][q] & 0xffffu), w1 = bf16_bits_to_f32(wv[i][q] >> 16);
      o[q] = (uint32_t)f32_to_bf16_bits(v[i][2 * q] * inv * w0) |
             ((uint32_t)f32_to_bf16_bits(v[i][2 * q + 1] * inv * w1) << 16);
    }
    orow[c] = o;
  }
}

// Gated RMSNorm of the Gated-DeltaNet output: per head of D values,
// out = rmsnorm(y) * w * silu(z), y fp32 or bf16, z bf16 (row stride ldz).
constexpr int kGatedPer = 16;  // values per lane: D <= 1024

// kN = D / 64 values per lane, a compile-time count so that the loads are straight-line code.
template <int kN>
__global__ __launch_bounds__(64) void gated_rmsnorm_kernel(const float* __restrict__ y, const uint16_t* __restrict__ z,
                                                           int ldz, const uint16_t* __restrict__ w, float eps,
                                                           uint16_t* __restrict__ out, int H) {
  // One wave per (token, head), lane i holding values i, i + 64, ..., i + 64 (kN - 1). Every load
  // is issued before the first is used: y, z and the weight together.
  constexpr int D = 64 * kN;
  const int t = blockIdx.y, h = blockIdx.x, lane = threadIdx.x;
  const float* yr = y + ((size_t)t * H + h) * D;
  const uint16_t* zr = z + (size_t)t * ldz + (size_t)h * D;
  float yv[kN];
  uint16_t zv[kN], wv[kN];
#pragma unroll
  for (int j = 0; j < kN; ++j) {
    yv[j] = yr[lane + 64 * j];
    zv[j] = zr[lane + 64 * j];
    wv[j] = w[lane + 64 * j];
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kN; ++j) ss = fmaf(yv[j], yv[j], ss);
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)D + eps);
#pragma unroll
  for (int j = 0; j < kN; ++j) {
    const float zf = bf16_bits_to_f32(zv[j]);
    const float gate = silu_gate(zf);
    out[((size_t)t * H + h) * D + lane + 64 * j] = f32_to_bf16_bits(yv[j] * inv * bf16_bits_to_f32(wv[j]) * gate);
  }
}

using GatedKernel = void (*)(const float*, const uint16_t*, int, const uint16_t*, float, uint16_t*, int);

template <int... kN>
constexpr auto gated_kernels(std::integer_sequence<int, kN...>) {
  return std::array<GatedKernel, sizeof...(kN)>{gated_rmsnorm_kernel<kN + 1>...};
}

}  // namespace

extern "C" int skinny_rmsnorm_bf16(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, float eps,
                                   uint16_t* out, uint16_t* sum_out, int rows, int H, void* stream) {
  SKINNY_CHECK_ARG(x && weight && out, "rmsnorm: null pointer");
  SKINNY_CHECK_ARG(rows >= 1 && H >= 8 && H % 8 == 0 && H <= 8 * kRowChunks * kThreads,
                   "rmsnorm: bad shape rows=%d H=%d (H must be a multiple of 8, at most %d)", rows, H,
                   8 * kRowChunks * kThreads);
  SKINNY_CHECK_ARG(skinny_aligned(x, 16) && skinny_aligned(weight, 16) && skinny_aligned(out, 16) &&
                       (!residual || skinny_aligned(residual, 16)) && (!sum_out || skinny_aligned(sum_out, 16)),
                   "rmsnorm: buffers must be 16-byte aligned");
  SKINNY_CHECK_ARG(!(sum_out && !residual), "rmsnorm: sum_out needs a residual");
  SKINNY_CHECK_ARG(out != x && out != residual, "rmsnorm: out must not alias the inputs");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, H, 0, x, residual, nullptr,
                     (size_t)0, 0, eps, weight, sum_out, out);
  return skinny_check_launch("rmsnorm");
}

extern "C" int skinny_mtp_input_bf16(const int32_t* ids, int tokens, const uint16_t* table, int V,
                                     const uint16_t* hidden, int ldh, const uint16_t* w_e, const uint16_t* w_h,
                                     float eps, uint16_t* out, int H, void* stream) {
  SKINNY_CHECK_ARG(ids && table && hidden && w_e && w_h && out, "mtp_input: null pointer");
  SKINNY_CHECK_ARG(tokens >= 1 && V >= 1 && H >= 8 && H % 8 == 0 && H <= 8 * kRowChunks * kThreads && ldh >= H &&
                       ldh % 8 == 0,
                   "mtp_input: bad shape tokens=%d V=%d H=%d ldh=%d", tokens, V, H, ldh);
  SKINNY_CHECK_ARG(skinny_aligned(table, 16) && skinny_aligned(hidden, 16) && skinny_aligned(w_e, 16) &&
                       skinny_aligned(w_h, 16) && skinny_aligned(out, 16),
                   "mtp_input: buffers must be 16-byte aligned");
  hipLaunchKernelGGL(mtp_input_kernel, dim3(2 * tokens), dim3(kThreads), 0, (hipStream_t)stream, H, tokens, ids, table,
                     V, hidden, ldh, w_e, w_h, eps, out);
  return skinny_check_launch("mtp_input");
}

extern "C" int skinny_rmsnorm_partials_bf16(const uint16_t* x, const float* parts, int splits, size_t split_stride,
                                            int ldp, const uint16_t* weight, float eps, uint16_t* out,
                                            uint16_t* sum_out, int rows, int H, void* stream) {
  SKINNY_CHECK_ARG(x && parts && weight && out, "rmsnorm partials: null pointer");
  SKINNY_CHECK_ARG(rows >= 1 && H >= 8 && H % 8 == 0 && H <= 8 * kRowChunks * kThreads,
                   "rmsnorm partials: bad shape rows=%d H=%d", rows, H);
  SKINNY_CHECK_ARG(splits >= 1 && splits <= kMaxSplits, "rmsnorm partials: splits=%d must be in [1, %d]", splits,
                   kMaxSplits);
  SKINNY_CHECK_ARG(ldp >= H && ldp % 4 == 0 && split_stride % 4 == 0 && split_stride >= (size_t)rows * ldp,
                   "rmsnorm partials: bad slice layout (ldp=%d, stride=%zu)", ldp, split_stride);
  SKINNY_CHECK_ARG(skinny_aligned(x, 16) && skinny_aligned(weight, 16) && skinny_aligned(out, 16) &&
                       skinny_aligned(parts, 16) && (!sum_out || skinny_aligned(sum_out, 16)),
                   "rmsnorm partials: buffers must be 16-byte aligned");
  SKINNY_CHECK_ARG(out != x, "rmsnorm partials: out must not alias x");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, H, splits, x, nullptr, parts,
                     split_stride, ldp, eps, weight, sum_out, out);
  return skinny_check_launch("rmsnorm partials");
}

extern "C" int skinny_gated_rmsnorm(const float* y, const uint16_t* z, int ldz, const uint16_t* weight, float eps,
                                    uint16_t* out, int tokens, int heads, int D, void* stream) {
  SKINNY_CHECK_ARG(y && z && weight && out, "gated_rmsnorm: null pointer");
  SKINNY_CHECK_ARG(tokens >= 1 && heads >= 1 && D >= 64 && D % 64 == 0 && D <= 64 * kGatedPer,
                   "gated_rmsnorm: D=%d must be a multiple of 64 in [64, %d]", D, 64 * kGatedPer);
  SKINNY_CHECK_ARG(ldz >= heads * D, "gated_rmsnorm: ldz=%d < heads*D", ldz);
  static constexpr auto kernels = gated_kernels(std::make_integer_sequence<int, kGatedPer>{});
  hipLaunchKernelGGL(kernels[D / 64 - 1], dim3(heads, tokens), dim3(64), 0, (hipStream_t)stream, y, z, ldz, weight, eps,
                     out, heads);
  return skinny_check_launch("gated_rmsnorm");
}
