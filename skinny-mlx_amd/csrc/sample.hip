// Sampling at temperature T > 0 and speculative rejection sampling, on the device.
//
// Reference: the reference decodes greedily (spec.py:137-147) and names rejection sampling for
// T > 0 as its next step (docs/flatspec-design.md:19, item F6; README.md:84). This is the
// standard speculative sampling (Leviathan et al. 2023; Chen et al. 2023): draft i is accepted
// with probability min(1, p_i(x)/q_i(x)); at the first rejection a sample of
// norm(max(0, p_i - q_i)) is emitted; if all K drafts are accepted, a sample of p_K. The emitted
// tokens are distributed exactly as sampling from the target alone.
//
// Random numbers are Philox4x32-10 (Salmon et al., SC 2011), keyed by the 64-bit seed, counter
// (n, stream): n = *counter + offset, read from device memory so a captured step draws fresh
// numbers on every replay. A uniform is the first output word's top 24 bits times 2^-24.
//
// Sampling is by inverse CDF over the vocabulary, deterministic: thread t of the workgroup owns
// the contiguous index range [t*c, (t+1)*c), sums its weights in index order, the chunk sums are
// scanned in a fixed order, and the thread whose interval holds u * total walks its range. Ties
// between claiming threads (possible only through rounding) go to the lowest thread.
#include "common.h"

namespace {

constexpr int kThreads = 1024;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ uint32_t philox_u32(uint64_t seed, uint64_t n, uint32_t stream) {
  uint32_t c0 = (uint32_t)n, c1 = (uint32_t)(n >> 32), c2 = stream, c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return c0;
}

__device__ __forceinline__ float uniform24(uint64_t seed, uint64_t n, uint32_t stream) {
  return (float)(philox_u32(seed, n, stream) >> 8) * 0x1p-24f;
}

// Workgroup-wide max and sum, fixed order (wave butterfly, then the waves in order).
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) t = fmaxf(t, red[w]);
  return t;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) t += red[w];
  return t;
}

__device__ __forceinline__ float piece_at(const u32x4_t& w, int e) {
  return bf16_bits_to_f32((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
}

// Rows are read in 16-byte pieces (8 logits) when 16-byte aligned, several loads in flight per
// thread; what is left one value at a time.
__device__ __forceinline__ float row_max(const uint16_t* row, int V, float* red) {
  float m = -INFINITY;
  const int nv = skinny_aligned(row, 16) ? V >> 3 : 0;
  const u32x4_t* r4 = reinterpret_cast<const u32x4_t*>(row);
#pragma unroll 4
  for (int i = threadIdx.x; i < nv; i += kThreads) {
    const u32x4_t w = r4[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, piece_at(w, e));
  }
  for (int i = 8 * nv + threadIdx.x; i < V; i += kThreads) m = fmaxf(m, bf16_bits_to_f32(row[i]));
  return block_max(m, red);
}

// Weights of 8 consecutive entries x0 .. x0+7 (x0 % 8 == 0) of a softmax row: exp((l - m) / T)
// from one 16-byte piece when the row is aligned, else per entry; entries at or past V weigh 0.
struct SoftmaxWeights {
  const uint16_t* row;
  int V;
  float m, c;
  bool vec;
  __device__ void operator()(int x0, float (&w)[8]) const {
    if (vec && x0 + 8 <= V) {
      const u32x4_t p = *reinterpret_cast<const u32x4_t*>(row + x0);
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = __builtin_amdgcn_exp2f((piece_at(p, e) - m) * c);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        w[e] = x0 + e < V ? __builtin_amdgcn_exp2f((bf16_bits_to_f32(row[x0 + e]) - m) * c) : 0.f;
    }
  }
};

struct SampleLds {
  float scan[kThreads];
  float red[kThreads / 64];
  int claim;
  int last_nz;
};

// Inverse-CDF sample of the non-negative weights of x in [0, V), with uniform u: the smallest x
// whose running sum exceeds u * total. weight8(x0, w) gives the weights of x0 .. x0+7 (zero past
// V); thread t owns [t*c, (t+1)*c) with c a multiple of 8. Returns -1 when every weight is zero.
template <class Weight8>
__device__ int inverse_cdf(const Weight8& weight8, int V, float u, SampleLds& s) {
  const int tid = threadIdx.x;
  const int chunk = ((V + kThreads - 1) / kThreads + 7) & ~7;
  const int lo = min(V, tid * chunk), hi = min(V, lo + chunk);
  float mine = 0.f;
#pragma unroll 4
  for (int x0 = lo; x0 < hi; x0 += 8) {
    float w[8];
    weight8(x0, w);
#pragma unroll
    for (int e = 0; e < 8; ++e) mine += w[e];
  }
  s.scan[tid] = mine;
  if (tid == 0) {
    s.claim = kThreads;
    s.last_nz = -1;
  }
  __syncthreads();
  for (int off = 1; off < kThreads; off <<= 1) {  // inclusive scan, fixed order
    const float v = tid >= off ? s.scan[tid - off] : 0.f;
    __syncthreads();
    s.scan[tid] += v;
    __syncthreads();
  }
  if (mine > 0.f) atomicMax(&s.last_nz, tid);
  __syncthreads();
  const float total = s.scan[kThreads - 1];
  const float thr = u * total;
  const float excl = tid ? s.scan[tid - 1] : 0.f, incl = s.scan[tid];
  const bool claims = mine > 0.f && excl <= thr && (thr < incl || tid == s.last_nz);
  if (claims) atomicMin(&s.claim, tid);
  __syncthreads();
  const int owner = s.claim;
  __syncthreads();
  if (owner == kThreads) return -1;
  if (tid == owner) {
    float acc = excl;
    int pick = -1, last = -1;
    for (int x0 = lo; x0 < hi && pick < 0; x0 += 8) {
      float w[8];
      weight8(x0, w);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (pick >= 0 || x0 + e >= hi) continue;
        if (w[e] > 0.f) last = x0 + e;
        acc += w[e];
        if (acc > thr && w[e] > 0.f) pick = x0 + e;
      }
    }
    s.claim = pick >= 0 ? pick : last;
  }
  __syncthreads();
  const int tok = s.claim;
  __syncthreads();
  return tok;
}

// One workgroup per row: token = inverse-CDF sample of softmax(row / T) with the uniform of
// counter *counter + offset + row, stream `rng_stream`.
__global__ __launch_bounds__(kThreads) void sample_rows_kernel(const uint16_t* __restrict__ logits, int V, int ld,
                                                               float inv_temp, uint64_t seed,
                                                               const int64_t* __restrict__ counter, int64_t offset,
                                                               uint32_t rng_stream, int32_t* __restrict__ out) {
  __shared__ SampleLds s;
  const uint16_t* row = logits + (size_t)blockIdx.x * ld;
  const float m = row_max(row, V, s.red);
  const float c = inv_temp * kLog2e;
  const float u = uniform24(seed, (uint64_t)(counter[0] + offset + blockIdx.x), rng_stream);
  const SoftmaxWeights w{row, V, m, c, skinny_aligned(row, 16)};
  const int tok = inverse_cdf(w, V, u, s);
  if (threadIdx.x == 0) out[blockIdx.x] = tok < 0 ? 0 : tok;
}

// stats[r] = (max, sum exp((x - max) / T)) of each row.
__global__ __launch_bounds__(kThreads) void row_stats_kernel(const uint16_t* __restrict__ logits, int V, int ld,
                                                             float inv_temp, float* __restrict__ stats) {
  __shared__ float red[kThreads / 64];
  const uint16_t* row = logits + (size_t)blockIdx.x * ld;
  const float m = row_max(row, V, red);
  const float c = inv_temp * kLog2e;
  float z = 0.f;
  const int nv = skinny_aligned(row, 16) ? V >> 3 : 0;
  const u32x4_t* r4 = reinterpret_cast<const u32x4_t*>(row);
#pragma unroll 4
  for (int i = threadIdx.x; i < nv; i += kThreads) {
    const u32x4_t w = r4[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) z += __builtin_amdgcn_exp2f((piece_at(w, e) - m) * c);
  }
  for (int i = 8 * nv + threadIdx.x; i < V; i += kThreads) z += __builtin_amdgcn_exp2f((bf16_bits_to_f32(row[i]) - m) * c);
  z = block_sum(z, red);
  if (threadIdx.x == 0) {
    stats[2 * blockIdx.x] = m;
    stats[2 * blockIdx.x + 1] = z;
  }
}

// One speculative step, one workgroup. target rows 0..K (stride ldt, stats_t), draft rows 0..K-1
// over the draft vocabulary [0, Vd) (stride ldd, stats_d), or none (draft == NULL: point-mass
// drafts). out = [n accepted, emitted token, n + 1].
__global__ __launch_bounds__(kThreads) void spec_accept_sampled_kernel(
    const uint16_t* __restrict__ target, int ldt, const float* __restrict__ stats_t, const uint16_t* __restrict__ draft,
    int ldd, const float* __restrict__ stats_d, int Vd, const int32_t* __restrict__ drafts, int K, int V,
    float inv_temp, uint64_t seed, const int64_t* __restrict__ counter, int32_t* __restrict__ out) {
  __shared__ SampleLds s;
  const float c = inv_temp * kLog2e;
  const uint64_t base = (uint64_t)counter[0];
  auto p_of = [&](int i, int x) {
    return __builtin_amdgcn_exp2f((bf16_bits_to_f32(target[(size_t)i * ldt + x]) - stats_t[2 * i]) * c) /
           stats_t[2 * i + 1];
  };
  auto q_of = [&](int i, int x) {
    if (!draft) return x == drafts[i] ? 1.0f : 0.0f;
    if (x >= Vd) return 0.0f;
    return __builtin_amdgcn_exp2f((bf16_bits_to_f32(draft[(size_t)i * ldd + x]) - stats_d[2 * i]) * c) /
           stats_d[2 * i + 1];
  };
  int n = K;
  bool rejected = false;
  for (int i = 0; i < K; ++i) {  // the same decisions in every thread
    const int x = drafts[i];
    const bool valid = x >= 0 && x < V;
    const float p = valid ? p_of(i, x) : 0.f;
    const float q = valid ? q_of(i, x) : 1.f;
    const float u = uniform24(seed, base + 2 * i, 0u);
    if (!(u * q < p)) {
      n = i;
      rejected = true;
      break;
    }
  }
  const float u2 = uniform24(seed, base + 2 * n + 1, 0u);
  // The emitted token's row: n (a rejection: the residual max(0, p - q)) or K (the bonus: p).
  const uint16_t* trow = target + (size_t)n * ldt;
  const SoftmaxWeights pw{trow, V, stats_t[2 * n], c, skinny_aligned(trow, 16)};
  int tok;
  if (rejected) {
    const float zt = stats_t[2 * n + 1];
    const uint16_t* drow = draft ? draft + (size_t)n * ldd : nullptr;
    const bool dvec = drow && skinny_aligned(drow, 16);
    const float md = draft ? stats_d[2 * n] : 0.f, zd = draft ? stats_d[2 * n + 1] : 1.f;
    const int xd = drafts[n];
    auto resid = [&](int x0, float (&w)[8]) {
      pw(x0, w);  // unnormalised p
      float q[8];
      if (!draft) {
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = x0 + e == xd ? 1.f : 0.f;
      } else if (dvec && x0 + 8 <= Vd) {
        const u32x4_t d = *reinterpret_cast<const u32x4_t*>(drow + x0);
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = __builtin_amdgcn_exp2f((piece_at(d, e) - md) * c) / zd;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          q[e] = x0 + e < Vd ? __builtin_amdgcn_exp2f((bf16_bits_to_f32(drow[x0 + e]) - md) * c) / zd : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = fmaxf(w[e] / zt - q[e], 0.f);
    };
    tok = inverse_cdf(resid, V, u2, s);
    if (tok < 0) tok = inverse_cdf(pw, V, u2, s);  // p == q to rounding everywhere: the target row itself
  } else {
    tok = inverse_cdf(pw, V, u2, s);
  }
  if (threadIdx.x == 0) {
    out[0] = n;
    out[1] = tok < 0 ? 0 : tok;
    out[2] = n + 1;
  }
}

__global__ void random_uniform_kernel(uint64_t seed, const int64_t* __restrict__ counter, int64_t offset, int n,
                                      uint32_t rng_stream, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = uniform24(seed, (uint64_t)(counter[0] + offset + i), rng_stream);
}

}  // namespace

extern "C" int skinny_random_uniform(uint64_t seed, const int64_t* counter, int64_t offset, int n, int rng_stream,
                                     float* out, void* stream) {
  SKINNY_CHECK_ARG(counter && out, "random_uniform: null pointer");
  SKINNY_CHECK_ARG(n >= 1 && rng_stream >= 0, "random_uniform: bad n=%d or stream=%d", n, rng_stream);
  hipLaunchKernelGGL(random_uniform_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, seed, counter,
                     offset, n, (uint32_t)rng_stream, out);
  return skinny_check_launch("random_uniform");
}

extern "C" int skinny_row_stats_bf16(const uint16_t* logits, int rows, int V, int ld, float inv_temp, float* stats,
                                     void* stream) {
  SKINNY_CHECK_ARG(logits && stats, "row_stats: null pointer");
  SKINNY_CHECK_ARG(rows >= 1 && V >= 1 && ld >= V && inv_temp > 0.f, "row_stats: bad shape or temperature");
  hipLaunchKernelGGL(row_stats_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, logits, V, ld, inv_temp,
                     stats);
  return skinny_check_launch("row_stats");
}

extern "C" int skinny_sample_rows_bf16(const uint16_t* logits, int rows, int V, int ld, float inv_temp, uint64_t seed,
                                       const int64_t* counter, int64_t offset, int rng_stream, int32_t* out,
                                       void* stream) {
  SKINNY_CHECK_ARG(logits && counter && out, "sample_rows: null pointer");
  SKINNY_CHECK_ARG(rows >= 1 && V >= 1 && ld >= V && inv_temp > 0.f && rng_stream >= 0,
                   "sample_rows: bad shape, temperature or stream");
  hipLaunchKernelGGL(sample_rows_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, logits, V, ld, inv_temp,
                     seed, counter, offset, (uint32_t)rng_stream, out);
  return skinny_check_launch("sample_rows");
}

extern "C" int skinny_spec_accept_sampled(const uint16_t* target, int ldt, const float* stats_t, const uint16_t* draft,
                                          int ldd, const float* stats_d, int Vd, const int32_t* drafts, int K, int V,
                                          float inv_temp, uint64_t seed, const int64_t* counter, int32_t* out,
                                          void* stream) {
  SKINNY_CHECK_ARG(target && stats_t && counter && out && (K == 0 || drafts), "spec_accept_sampled: null pointer");
  SKINNY_CHECK_ARG(!draft || stats_d, "spec_accept_sampled: draft rows need their stats");
  SKINNY_CHECK_ARG(K >= 0 && V >= 1 && ldt >= V && inv_temp > 0.f, "spec_accept_sampled: bad shape or temperature");
  SKINNY_CHECK_ARG(!draft || (Vd >= 1 && Vd <= V && ldd >= Vd), "spec_accept_sampled: bad draft vocabulary");
  hipLaunchKernelGGL(spec_accept_sampled_kernel, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, target, ldt, stats_t,
                     draft, ldd, stats_d, Vd, drafts, K, V, inv_temp, seed, counter, out);
  return skinny_check_launch("spec_accept_sampled");
}
