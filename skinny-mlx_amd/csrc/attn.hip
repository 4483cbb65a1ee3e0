// Full attention of the verify step: M <= 16 new tokens against a KV cache, GQA.
//
// Reference behaviour: the full-attention layers of the mlx_lm decoder the reference
// patches (skinny_mlx/spec.py:24-29 runs them through `model(...)`; KVCache append/trim at
// spec.py:78, 93 and rollback.py:71-73), with per-head q/k RMSNorm and rotate-half RoPE.
//
// Cache layout (per layer): K [Hkv][maxlen][D] and V transposed, Vt [Hkv][D][maxlen], bf16.
// The transposed V makes eight consecutive keys of one dimension contiguous — exactly the
// B operand of the P.V MFMA. The number of tokens already cached (`pos0`) is read from
// device memory, so a launch sequence can be captured once and replayed at any length.
//
// Every query row is computed from its own data only and every reduction runs in a fixed
// order over absolute key positions (chunks of 128 keys), so a token's output
// does not depend on how many tokens share the step.
#include <mutex>

#include "attn_chunk.h"

namespace {

// --- q/k RMSNorm + RoPE + cache store ---------------------------------------------------------

// One wave per (head, token). Heads [0, Hq) are queries (written to q_out), [Hq, Hq+Hkv) keys
// (written to the K cache at slot pos0 + t), [Hq+Hkv, Hq+2Hkv) values (to Vt). Token t is rotated
// to position pos0 + t, or pos0 + rpos[t] for a draft tree (its depth).
__global__ __launch_bounds__(64) void qk_rope_store_kernel(const uint16_t* __restrict__ qkv, int ldq, int Hq, int Hkv,
                                                           const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn,
                                                           float eps, const int32_t* __restrict__ pos0, float theta,
                                                           const int32_t* __restrict__ tree, int M,
                                                           uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                                           uint16_t* __restrict__ vt, int maxlen) {
  const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const int slot = pos0[0] + t;                                 // cache slot of token t
  const int pos = pos0[0] + (tree ? tree[1 + M + t] : t);       // its RoPE position
  const uint16_t* src = qkv + (size_t)t * ldq + (size_t)head * kD;
  float a = bf16_bits_to_f32(src[lane]), b = bf16_bits_to_f32(src[lane + 64]);
  if (head >= Hq + Hkv) {  // value: straight into the transposed cache
    const int h = head - Hq - Hkv;
    vt[((size_t)h * kD + lane) * maxlen + slot] = src[lane];
    vt[((size_t)h * kD + lane + 64) * maxlen + slot] = src[lane + 64];
    return;
  }
  const uint16_t* nw = head < Hq ? qn : kn;
  if (nw) {
    const float ss = wave_sum(fmaf(b, b, a * a));
    const float inv = rsqrtf(ss / (float)kD + eps);
    a = bf16_bits_to_f32(f32_to_bf16_bits(a * inv * bf16_bits_to_f32(nw[lane])));
    b = bf16_bits_to_f32(f32_to_bf16_bits(b * inv * bf16_bits_to_f32(nw[lane + 64])));
  }
  // rotate-half RoPE on the pair (i, i + D/2), frequency theta^(-2i/D)
  const float inv_freq = powf(theta, -2.0f * (float)lane / (float)kD);
  float sn, cs;
  sincosf((float)pos * inv_freq, &sn, &cs);
  // explicit fused multiply-adds, the same in the fused attention kernel: its key rows are these bits
  const uint16_t ra = f32_to_bf16_bits(fmaf(a, cs, -(b * sn)));
  const uint16_t rb = f32_to_bf16_bits(fmaf(b, cs, a * sn));
  if (head < Hq) {
    uint16_t* dst = q_out + ((size_t)t * Hq + head) * kD;
    dst[lane] = ra;
    dst[lane + 64] = rb;
  } else {
    uint16_t* dst = kc + ((size_t)(head - Hq) * maxlen + slot) * kD;
    dst[lane] = ra;
    dst[lane + 64] = rb;
  }
}


// The device position comes first among the arguments: it is the kernel's first read, and the
// leading argument dwords arrive preloaded in SGPRs.
template <bool kFused>
__global__ __launch_bounds__(64 * kWaves) void attn_chunk_kernel(const int32_t* __restrict__ pos0,
                                                                 const uint16_t* __restrict__ q, FusedArgs fa, int M,
                                                                 int Hq, int Hkv, uint16_t* __restrict__ kc,
                                                                 uint16_t* __restrict__ vt, int maxlen, float scale,
                                                                 const int32_t* __restrict__ tree,
                                                                 float* __restrict__ part_o, float* __restrict__ part_ml,
                                                                 int nchunk_max) {
  attn_chunk_body<kFused>((int)blockIdx.x, (int)blockIdx.y, pos0, q, fa, M, Hq, Hkv, kc, vt, maxlen, scale, tree, part_o,
                          part_ml, nchunk_max);
}

// One workgroup per (q head, token): merge the chunk partials, normalise, store bf16. Chunks are
// taken in blocks of 32 by absolute index: all of a block's loads are issued together (lane c holds
// chunk c's statistics, every lane its two dims of every chunk's partial row), then the block is
// folded into running sums in chunk order, rescaled when the running maximum grows. A block past
// a row's position holds only empty chunks and rescales by exactly 1, so the result does not
// depend on how many tokens share the step. With W waves (caches of more than one block), wave v
// folds blocks v, v + W, ... into sums of its own, and wave 0 then folds waves 1 .. W-1 into its
// sums in that order, a wave without keys for the row by exactly 1 and 0: W is fixed by the cache
// size, so every step over one cache merges a row's blocks the same way.
constexpr int kCombineBlock = 32;
constexpr int kCombineWaves = 4;  // waves of the merge for caches of more than kCombineBlock chunks

template <int W>
__global__ __launch_bounds__(64 * W) void attn_combine_kernel(const float* __restrict__ part_o,
                                                              const float* __restrict__ part_ml, int M, int Hq, int Hkv,
                                                              const int32_t* __restrict__ pos0, int nchunk_max,
                                                              uint16_t* __restrict__ out, uint32_t* __restrict__ reset,
                                                              int reset_ld, int reset_words) {
  const int hq = blockIdx.x, t = blockIdx.y, lane = threadIdx.x & 63, v = W > 1 ? wave_id() : 0;
  const int G = Hq / Hkv, h = hq / G, row = t * G + hq % G;
  const size_t head_base = (size_t)h * nchunk_max * kRowsMax + row;  // chunk c at + c * kRowsMax
  const int first = v * kCombineBlock;                                // this wave's first block
  // The first block's partials are loaded before the chunk count is known (it needs *pos0):
  // every chunk the workspace holds up to kCombineBlock, the ones past the context discarded below
  // by selection (their stale values never enter an arithmetic operation).
  const int pre = max(0, min(kCombineBlock, nchunk_max - first));
  float mc_pre = -INFINITY, lc_pre = 0.f;
  float o0[kCombineBlock], o1[kCombineBlock];
  if (lane < pre) {
    mc_pre = part_ml[(head_base + (size_t)(first + lane) * kRowsMax) * 2];
    lc_pre = part_ml[(head_base + (size_t)(first + lane) * kRowsMax) * 2 + 1];
  }
#pragma unroll
  for (int j = 0; j < kCombineBlock; ++j) {
    o0[j] = o1[j] = 0.f;
    if (j < pre) {
      const float* po = part_o + (head_base + (size_t)(first + j) * kRowsMax) * kD;
      o0[j] = po[lane];
      o1[j] = po[lane + 64];
    }
  }
  const int total = pos0[0] + M;
  const int nch = (total + kChunk - 1) / kChunk;
  float run_m = -INFINITY, run_l = 0.f, a0 = 0.f, a1 = 0.f;
  for (int c0 = first; c0 < nch; c0 += W * kCombineBlock) {
    const int nb = min(kCombineBlock, nch - c0);
    float mc = -INFINITY, lc = 0.f;
    if (c0 == first) {
      mc = lane < nb ? mc_pre : -INFINITY;
      lc = lane < nb ? lc_pre : 0.f;
#pragma unroll
      for (int j = 0; j < kCombineBlock; ++j) {
        o0[j] = j < nb ? o0[j] : 0.f;
        o1[j] = j < nb ? o1[j] : 0.f;
      }
    } else {
      if (lane < nb) {
        mc = part_ml[(head_base + (size_t)(c0 + lane) * kRowsMax) * 2];
        lc = part_ml[(head_base + (size_t)(c0 + lane) * kRowsMax) * 2 + 1];
      }
#pragma unroll
      for (int j = 0; j < kCombineBlock; ++j) {
        o0[j] = o1[j] = 0.f;
        if (j < nb) {
          const float* po = part_o + (head_base + (size_t)(c0 + j) * kRowsMax) * kD;
          o0[j] = po[lane];
          o1[j] = po[lane + 64];
        }
      }
    }
    float bm = mc;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) bm = fmaxf(bm, __shfl_xor(bm, off, 64));
    const float new_m = fmaxf(run_m, bm);
    const float keep = run_m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(run_m - new_m);
    run_l *= keep;
    a0 *= keep;
    a1 *= keep;
    const float wgt = mc == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc - new_m);
#pragma unroll
    for (int j = 0; j < kCombineBlock; ++j) {
      if (j < nb) {  // lane j's weight and sum, broadcast by v_readlane (j is a constant here)
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), j));
        run_l = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(lc), j)), wj, run_l);
        a0 = fmaf(o0[j], wj, a0);
        a1 = fmaf(o1[j], wj, a1);
      }
    }
    run_m = new_m;
  }
  if constexpr (W > 1) {
    __shared__ float sm[W], sl[W], sa[W][2][64];
    if (lane == 0) {
      sm[v] = run_m;
      sl[v] = run_l;
    }
    sa[v][0][lane] = a0;
    sa[v][1][lane] = a1;
    __syncthreads();
    if (v > 0) return;
#pragma unroll
    for (int u = 1; u < W; ++u) {
      const float mu = sm[u], lu = sl[u];
      const float new_m = fmaxf(run_m, mu);
      const float k0 = run_m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(run_m - new_m);
      const float ku = mu == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mu - new_m);
      run_l = fmaf(lu, ku, run_l * k0);
      a0 = fmaf(sa[u][0][lane], ku, a0 * k0);
      a1 = fmaf(sa[u][1][lane], ku, a1 * k0);
      run_m = new_m;
    }
  }
  const float inv = run_l > 0.f ? 1.0f / run_l : 0.f;
  uint16_t* dst = out + ((size_t)t * Hq + hq) * kD;
  dst[lane] = f32_to_bf16_bits(a0 * inv);
  dst[lane + 64] = f32_to_bf16_bits(a1 * inv);
  if (reset) {  // every chunk workgroup has read the hand-off rows: back to "not yet written"
    const int per = (reset_words + Hq - 1) / Hq;
    const int w1 = min(reset_words, (hq + 1) * per);
    uint32_t* r = reset + (size_t)t * reset_ld;
    for (int w = hq * per + lane; w < w1; w += 64)
      __hip_atomic_store(r + w, 0xffffffffu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// cos/sin table of rotate-half RoPE: table[pos][i] = (cos, sin)(pos * theta^(-2i/128)), i < 64,
// by the same expressions as qk_rope_store_kernel.
__global__ void rope_table_kernel(float theta, int positions, float* __restrict__ table) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= positions * 64) return;
  const int pos = idx >> 6, i = idx & 63;
  const float inv_freq = powf(theta, -2.0f * (float)i / (float)kD);
  float sn, cs;
  sincosf((float)pos * inv_freq, &sn, &cs);
  table[2 * idx] = cs;
  table[2 * idx + 1] = sn;
}

}  // namespace

int attn_combine_launch(const float* part_o, const float* part_ml, int M, int Hq, int Hkv, const int32_t* pos0,
                        int nchunk_max, uint16_t* out, uint32_t* reset, int reset_ld, int reset_words,
                        hipStream_t stream) {
  if (nchunk_max > kCombineBlock)
    hipLaunchKernelGGL(attn_combine_kernel<kCombineWaves>, dim3(Hq, M), dim3(64 * kCombineWaves), 0, stream, part_o,
                       part_ml, M, Hq, Hkv, pos0, nchunk_max, out, reset, reset_ld, reset_words);
  else
    hipLaunchKernelGGL(attn_combine_kernel<1>, dim3(Hq, M), dim3(64), 0, stream, part_o, part_ml, M, Hq, Hkv, pos0,
                       nchunk_max, out, reset, reset_ld, reset_words);
  return skinny_check_launch("attention combine");
}

extern "C" int skinny_rope_table(float theta, int positions, float* table, void* stream) {
  SKINNY_CHECK_ARG(table && positions >= 1 && theta > 1.f, "rope_table: bad arguments");
  hipLaunchKernelGGL(rope_table_kernel, dim3((positions * 64 + 255) / 256), dim3(256), 0, (hipStream_t)stream, theta,
                     positions, table);
  return skinny_check_launch("rope_table");
}

extern "C" int skinny_qk_rope_store(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D,
                                    const uint16_t* q_norm, const uint16_t* k_norm, float eps, const int32_t* pos0,
                                    float theta, const int32_t* tree, uint16_t* q_out, uint16_t* k_cache,
                                    uint16_t* vt_cache, int maxlen, void* stream) {
  SKINNY_CHECK_ARG(qkv && pos0 && q_out && k_cache && vt_cache, "qk_rope_store: null pointer");
  SKINNY_CHECK_ARG(D == kD, "qk_rope_store: head dim %d unsupported (only %d)", D, kD);
  SKINNY_CHECK_ARG(M >= 1 && M <= 65535 && Hq >= 1 && Hkv >= 1 && Hq % Hkv == 0, "qk_rope_store: bad heads/tokens");
  SKINNY_CHECK_ARG(ldq >= (Hq + 2 * Hkv) * D, "qk_rope_store: ldq=%d too small", ldq);
  SKINNY_CHECK_ARG(maxlen >= 1, "qk_rope_store: bad maxlen");
  SKINNY_CHECK_ARG(!tree || M <= 32, "qk_rope_store: a draft tree holds at most 32 tokens (M=%d)", M);
  hipLaunchKernelGGL(qk_rope_store_kernel, dim3(Hq + 2 * Hkv, M), dim3(64), 0, (hipStream_t)stream, qkv, ldq, Hq, Hkv,
                     q_norm, k_norm, eps, pos0, theta, tree, M, q_out, k_cache, vt_cache, maxlen);
  return skinny_check_launch("qk_rope_store");
}

extern "C" size_t skinny_attn_workspace_bytes(int Hkv, int maxlen) {
  const size_t nch = (size_t)((maxlen + kChunk - 1) / kChunk);
  return (size_t)Hkv * nch * kRowsMax * (kD + 2) * sizeof(float);
}

extern "C" int skinny_attention_bf16(const uint16_t* q, int M, int Hq, int Hkv, int D, const uint16_t* k_cache,
                                     const uint16_t* vt_cache, int maxlen, const int32_t* pos0, float scale,
                                     const int32_t* tree, float* workspace, size_t workspace_bytes, uint16_t* out,
                                     void* stream) {
  SKINNY_CHECK_ARG(q && k_cache && vt_cache && pos0 && workspace && out, "attention: null pointer");
  SKINNY_CHECK_ARG(D == kD, "attention: head dim %d unsupported (only %d)", D, kD);
  SKINNY_CHECK_ARG(Hkv >= 1 && Hq % Hkv == 0, "attention: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  SKINNY_CHECK_ARG(M >= 1 && (Hq / Hkv) * M <= kRowsMax, "attention: %d query rows per kv head exceed %d",
                   (Hq / Hkv) * M, kRowsMax);
  SKINNY_CHECK_ARG(maxlen >= kChunk && maxlen % kChunk == 0, "attention: maxlen=%d must be a multiple of %d", maxlen,
                   kChunk);
  SKINNY_CHECK_ARG(workspace_bytes >= skinny_attn_workspace_bytes(Hkv, maxlen), "attention: workspace too small");
  SKINNY_CHECK_ARG(skinny_aligned(q, 16) && skinny_aligned(k_cache, 16) && skinny_aligned(vt_cache, 16),
                   "attention: q and caches must be 16-byte aligned");
  const int nch = maxlen / kChunk;
  float* part_o = workspace;
  float* part_ml = workspace + (size_t)Hkv * nch * kRowsMax * kD;
  const FusedArgs none{0, nullptr, nullptr, 0.f, nullptr};
  hipLaunchKernelGGL(attn_chunk_kernel<false>, dim3(nch, Hkv), dim3(64 * kWaves), 0, (hipStream_t)stream, pos0, q, none, M,
                     Hq, Hkv, const_cast<uint16_t*>(k_cache), const_cast<uint16_t*>(vt_cache), maxlen, scale, tree,
                     part_o, part_ml, nch);
  int rc = skinny_check_launch("attention");
  if (rc) return rc;
  return attn_combine_launch(part_o, part_ml, M, Hq, Hkv, pos0, nch, out, nullptr, 0, 0, (hipStream_t)stream);
}

// Validation and launches of the fused attention, given the chunk-partial workspace.
static int attention_fused(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D, const uint16_t* q_norm,
                           const uint16_t* k_norm, float eps, const float* rope_table, int rope_positions,
                           const int32_t* pos0, const int32_t* tree, uint16_t* k_cache, uint16_t* vt_cache,
                           int maxlen, float scale, float* workspace, size_t workspace_bytes, uint16_t* out,
                           void* stream) {
  SKINNY_CHECK_ARG(qkv && rope_table && k_cache && vt_cache && pos0 && workspace && out, "attention: null pointer");
  SKINNY_CHECK_ARG(D == kD, "attention: head dim %d unsupported (only %d)", D, kD);
  SKINNY_CHECK_ARG(Hkv >= 1 && Hq % Hkv == 0, "attention: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  SKINNY_CHECK_ARG(M >= 1 && M <= kFusedMaxTokens && (Hq / Hkv) * M <= kRowsMax,
                   "attention: M=%d (at most %d) with %d query rows per kv head (at most %d)", M, kFusedMaxTokens,
                   (Hq / Hkv) * M, kRowsMax);
  SKINNY_CHECK_ARG(ldq >= (Hq + 2 * Hkv) * D && ldq % 8 == 0, "attention: ldq=%d too small or not a multiple of 8",
                   ldq);
  SKINNY_CHECK_ARG(maxlen >= kChunk && maxlen % kChunk == 0 && rope_positions >= maxlen,
                   "attention: maxlen=%d must be a multiple of %d and within the RoPE table (%d)", maxlen, kChunk,
                   rope_positions);
  SKINNY_CHECK_ARG(workspace_bytes >= skinny_attn_workspace_bytes(Hkv, maxlen), "attention: workspace too small");
  SKINNY_CHECK_ARG(skinny_aligned(qkv, 16) && skinny_aligned(k_cache, 16) && skinny_aligned(vt_cache, 16) &&
                       skinny_aligned(rope_table, 16) && (!q_norm || skinny_aligned(q_norm, 16)),
                   "attention: qkv, caches, table and q_norm must be 16-byte aligned");
  const int nch = maxlen / kChunk;
  float* part_o = workspace;
  float* part_ml = workspace + (size_t)Hkv * nch * kRowsMax * kD;
  const FusedArgs fa{ldq, q_norm, k_norm, eps, rope_table};
  hipLaunchKernelGGL(attn_chunk_kernel<true>, dim3(nch, Hkv), dim3(64 * kWaves), 0, (hipStream_t)stream, pos0, qkv, fa, M,
                     Hq, Hkv, k_cache, vt_cache, maxlen, scale, tree, part_o, part_ml, nch);
  int rc = skinny_check_launch("attention");
  if (rc) return rc;
  return attn_combine_launch(part_o, part_ml, M, Hq, Hkv, pos0, nch, out, nullptr, 0, 0, (hipStream_t)stream);
}

extern "C" int skinny_attention_fused_bf16(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D,
                                           const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                           const float* rope_table, int rope_positions, const int32_t* pos0,
                                           const int32_t* tree, uint16_t* k_cache, uint16_t* vt_cache, int maxlen,
                                           float scale, float* workspace, size_t workspace_bytes, uint16_t* out,
                                           void* stream) {
  return attention_fused(qkv, ldq, M, Hq, Hkv, D, q_norm, k_norm, eps, rope_table, rope_positions, pos0, tree,
                         k_cache, vt_cache, maxlen, scale, workspace, workspace_bytes, out, stream);
}

// --- the allocation-free form -----------------------------------------------------------------

// The chunk partials of skinny_attention_fused_noalloc_bf16: a file-scope device array (one copy
// per GPU, held until the process ends) instead of a caller workspace, sized for at most
// kScratchChunks (kv head, 128-key chunk) pairs — 8 kv heads over 4096 cached positions, 8.1 MiB.
// No entry needs it cleared: the chunk kernel writes every partial the combine kernel reads.
constexpr int kScratchChunks = 256;
constexpr size_t kScratchFloats = (size_t)kScratchChunks * kRowsMax * (kD + 2);
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device: in host code the
// array's name is only a stand-in, and every GPU holds its copy at its own address.
static int scratch_of_current_device(void* stream, float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return skinny_set_error(SKINNY_ELAUNCH, "attention (no alloc): hipGetDevice: %s", hipGetErrorString(e));
  if (stream) {
    hipDevice_t sdev = 0;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess)
      return skinny_set_error(SKINNY_ELAUNCH, "attention (no alloc): hipStreamGetDevice: %s", hipGetErrorString(e));
    SKINNY_CHECK_ARG((int)sdev == dev, "attention (no alloc): the stream is on device %d, the current device is %d",
                     (int)sdev, dev);
  }
  SKINNY_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "attention (no alloc): device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return skinny_set_error(SKINNY_ELAUNCH, "attention (no alloc): hipGetSymbolAddress(scratch) on device %d: %s", dev,
                              hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return SKINNY_OK;
}

extern "C" int skinny_attention_fused_noalloc_bf16(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D,
                                                   const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                                   const float* rope_table, int rope_positions, const int32_t* pos0,
                                                   const int32_t* tree, uint16_t* k_cache, uint16_t* vt_cache,
                                                   int maxlen, float scale, uint16_t* out, void* stream) {
  SKINNY_CHECK_ARG(Hkv >= 1 && maxlen >= kChunk && maxlen % kChunk == 0,
                   "attention (no alloc): Hkv=%d, maxlen=%d must be a multiple of %d", Hkv, maxlen, kChunk);
  SKINNY_CHECK_ARG((size_t)Hkv * (maxlen / kChunk) <= (size_t)kScratchChunks,
                   "attention (no alloc): %d kv heads x %d cached positions exceed the scratch maximum of %d "
                   "(kv head, %d-position chunk) pairs",
                   Hkv, maxlen, kScratchChunks, kChunk);
  float* ws = nullptr;
  if (int rc = scratch_of_current_device(stream, &ws)) return rc;
  return attention_fused(qkv, ldq, M, Hq, Hkv, D, q_norm, k_norm, eps, rope_table, rope_positions, pos0, tree,
                         k_cache, vt_cache, maxlen, scale, ws, kScratchFloats * sizeof(float), out, stream);
}
