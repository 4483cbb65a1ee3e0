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
// order over absolute key positions (waves of 32 keys, chunks of 256), so a token's output
// does not depend on how many tokens share the step.
#include "common.h"

namespace {

constexpr int kD = 128;             // head dim
constexpr int kWaves = 8;           // waves per workgroup, 32 keys each
constexpr int kChunk = 32 * kWaves;  // keys per workgroup
constexpr int kRowsMax = 64;        // GQA group (<= 4) x M (<= 16)

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// --- q/k RMSNorm + RoPE + cache store ---------------------------------------------------------

// One wave per (head, token). Heads [0, Hq) are queries (written to q_out), [Hq, Hq+Hkv) keys
// (written to the K cache at position pos0 + t), [Hq+Hkv, Hq+2Hkv) values (to Vt).
__global__ __launch_bounds__(64) void qk_rope_store_kernel(const uint16_t* __restrict__ qkv, int ldq, int Hq, int Hkv,
                                                           const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn,
                                                           float eps, const int32_t* __restrict__ pos0, float theta,
                                                           uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                                           uint16_t* __restrict__ vt, int maxlen) {
  const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const int pos = pos0[0] + t;
  const uint16_t* src = qkv + (size_t)t * ldq + (size_t)head * kD;
  float a = bf16_bits_to_f32(src[lane]), b = bf16_bits_to_f32(src[lane + 64]);
  if (head >= Hq + Hkv) {  // value: straight into the transposed cache
    const int h = head - Hq - Hkv;
    vt[((size_t)h * kD + lane) * maxlen + pos] = src[lane];
    vt[((size_t)h * kD + lane + 64) * maxlen + pos] = src[lane + 64];
    return;
  }
  const uint16_t* nw = head < Hq ? qn : kn;
  if (nw) {
    float ss = a * a + b * b;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float inv = rsqrtf(ss / (float)kD + eps);
    a = bf16_bits_to_f32(f32_to_bf16_bits(a * inv * bf16_bits_to_f32(nw[lane])));
    b = bf16_bits_to_f32(f32_to_bf16_bits(b * inv * bf16_bits_to_f32(nw[lane + 64])));
  }
  // rotate-half RoPE on the pair (i, i + D/2), frequency theta^(-2i/D)
  const float inv_freq = powf(theta, -2.0f * (float)lane / (float)kD);
  float sn, cs;
  sincosf((float)pos * inv_freq, &sn, &cs);
  const uint16_t ra = f32_to_bf16_bits(a * cs - b * sn);
  const uint16_t rb = f32_to_bf16_bits(b * cs + a * sn);
  if (head < Hq) {
    uint16_t* dst = q_out + ((size_t)t * Hq + head) * kD;
    dst[lane] = ra;
    dst[lane + 64] = rb;
  } else {
    uint16_t* dst = kc + ((size_t)(head - Hq) * maxlen + pos) * kD;
    dst[lane] = ra;
    dst[lane + 64] = rb;
  }
}

// --- chunked attention ------------------------------------------------------------------------

// Workgroup (chunk c, kv head h): keys [256c, 256c + 256), wave w owns 32 of them. For each
// 16-row tile of the (token, group head) rows: S = Q K^T by MFMA, causal mask on absolute
// positions, softmax statistics of the wave, P V by MFMA; the 8 wave partials are merged in
// wave order through LDS and written as the chunk partial (unnormalised O, max, sum).
__global__ __launch_bounds__(64 * kWaves) void attn_chunk_kernel(const uint16_t* __restrict__ q, int M, int Hq, int Hkv,
                                                                 const uint16_t* __restrict__ kc,
                                                                 const uint16_t* __restrict__ vt, int maxlen,
                                                                 const int32_t* __restrict__ pos0, float scale,
                                                                 float* __restrict__ part_o, float* __restrict__ part_ml,
                                                                 int nchunk_max) {
  const int c = blockIdx.x, h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p0 = pos0[0];
  const int total = p0 + M;  // keys present after this step's tokens were stored
  if (c * kChunk >= total) return;
  const int G = Hq / Hkv;
  const int rows = G * M;
  const int rtiles = (rows + 15) >> 4;
  const int key0 = c * kChunk + wave * 32;  // this wave's first key
  const int col = lane & 15, quad = lane >> 4;

  // K^T fragments (B operand of S = Q K^T): key tile kt, d step ks
  bf16x8_t kf[2][4];
  const uint16_t* kh = kc + (size_t)h * maxlen * kD;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      kf[kt][ks] = *reinterpret_cast<const bf16x8_t*>(kh + (size_t)(key0 + kt * 16 + col) * kD + ks * 32 + quad * 8);
  // V fragments (B operand of O = P V): d tile dt, keys key0 + 8quad + 0..7
  bf16x8_t vf[8];
  const uint16_t* vh = vt + (size_t)h * kD * maxlen;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    vf[dt] = *reinterpret_cast<const bf16x8_t*>(vh + (size_t)(dt * 16 + col) * maxlen + key0 + quad * 8);

  __shared__ uint16_t pbuf[kWaves][16][32];
  __shared__ float wo[kWaves][16][kD + 2];

  for (int rt = 0; rt < rtiles; ++rt) {
    // Q fragments (A operand): row rt*16 + col
    const int arow = rt * 16 + col;
    bf16x8_t qf[4];
    if (arow < rows) {
      const int t = arow / G, j = arow % G;
      const uint16_t* qr = q + ((size_t)t * Hq + h * G + j) * kD;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const bf16x8_t*>(qr + ks * 32 + quad * 8);
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qf[ks] = bf16x8_t{};
    }
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    float s[2][4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f32x4_t acc = zero;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc = mfma16x16x32(qf[ks], kf[kt][ks], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[kt][i] = acc[i];
    }
    // this lane's rows: rt*16 + 4quad + i ; key: key0 + 16kt + col
    float m[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = rt * 16 + quad * 4 + i;
      const int qpos = row < rows ? p0 + row / G : -1;
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int kp = key0 + kt * 16 + col;
        s[kt][i] = kp <= qpos ? s[kt][i] * scale : -INFINITY;
        mx = fmaxf(mx, s[kt][i]);
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      float sum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const float pv = s[kt][i] == -INFINITY ? 0.f : expf(s[kt][i] - mx);
        const uint16_t pb = f32_to_bf16_bits(pv);
        sum += bf16_bits_to_f32(pb);  // the sum matches the bf16 P that multiplies V
        pbuf[wave][quad * 4 + i][kt * 16 + col] = pb;
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) sum += __shfl_xor(sum, o, 64);
      m[i] = mx;
      l[i] = sum;
    }
    __syncthreads();
    const bf16x8_t pf = *reinterpret_cast<const bf16x8_t*>(&pbuf[wave][col][quad * 8]);
    f32x4_t o[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = mfma16x16x32(pf, vf[dt], zero);
    // wave partial -> LDS
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = quad * 4 + i;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) wo[wave][r][dt * 16 + col] = o[dt][i];
      if (col == 0) {
        wo[wave][r][kD] = m[i];
        wo[wave][r][kD + 1] = l[i];
      }
    }
    __syncthreads();
    // merge the waves in order: 16 rows x 128 dims over 512 threads, 4 each
    for (int e = threadIdx.x; e < 16 * kD; e += 64 * kWaves) {
      const int r = e / kD, d = e % kD;
      float mm = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, wo[w][r][kD]);
      float acc = 0.f, ls = 0.f;
      if (mm != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const float mw = wo[w][r][kD];
          if (mw == -INFINITY) continue;
          const float f = expf(mw - mm);
          acc = fmaf(wo[w][r][d], f, acc);
          ls = fmaf(wo[w][r][kD + 1], f, ls);
        }
      }
      const int row = rt * 16 + r;
      const size_t base = (((size_t)h * nchunk_max + c) * kRowsMax + row);
      part_o[base * kD + d] = acc;
      if (d == 0) {
        part_ml[base * 2] = mm;
        part_ml[base * 2 + 1] = ls;
      }
    }
    __syncthreads();
  }
}

// One wave per (q head, token): merge the chunk partials in chunk order, normalise, store bf16.
__global__ __launch_bounds__(64) void attn_combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                                          int M, int Hq, int Hkv, const int32_t* __restrict__ pos0,
                                                          int nchunk_max, uint16_t* __restrict__ out) {
  const int hq = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const int G = Hq / Hkv, h = hq / G, row = t * G + hq % G;
  const int total = pos0[0] + M;
  const int nch = (total + kChunk - 1) / kChunk;
  float mm = -INFINITY;
  for (int c = 0; c < nch; ++c) mm = fmaxf(mm, part_ml[(((size_t)h * nchunk_max + c) * kRowsMax + row) * 2]);
  float a0 = 0.f, a1 = 0.f, ls = 0.f;
  for (int c = 0; c < nch; ++c) {
    const size_t base = ((size_t)h * nchunk_max + c) * kRowsMax + row;
    const float mc = part_ml[base * 2];
    if (mc == -INFINITY) continue;
    const float f = expf(mc - mm);
    ls = fmaf(part_ml[base * 2 + 1], f, ls);
    a0 = fmaf(part_o[base * kD + lane], f, a0);
    a1 = fmaf(part_o[base * kD + lane + 64], f, a1);
  }
  const float inv = ls > 0.f ? 1.0f / ls : 0.f;
  uint16_t* dst = out + ((size_t)t * Hq + hq) * kD;
  dst[lane] = f32_to_bf16_bits(a0 * inv);
  dst[lane + 64] = f32_to_bf16_bits(a1 * inv);
}

}  // namespace

extern "C" int skinny_qk_rope_store(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D,
                                    const uint16_t* q_norm, const uint16_t* k_norm, float eps, const int32_t* pos0,
                                    float theta, uint16_t* q_out, uint16_t* k_cache, uint16_t* vt_cache, int maxlen,
                                    void* stream) {
  SKINNY_CHECK_ARG(qkv && pos0 && q_out && k_cache && vt_cache, "qk_rope_store: null pointer");
  SKINNY_CHECK_ARG(D == kD, "qk_rope_store: head dim %d unsupported (only %d)", D, kD);
  SKINNY_CHECK_ARG(M >= 1 && M <= 65535 && Hq >= 1 && Hkv >= 1 && Hq % Hkv == 0, "qk_rope_store: bad heads/tokens");
  SKINNY_CHECK_ARG(ldq >= (Hq + 2 * Hkv) * D, "qk_rope_store: ldq=%d too small", ldq);
  SKINNY_CHECK_ARG(maxlen >= 1, "qk_rope_store: bad maxlen");
  hipLaunchKernelGGL(qk_rope_store_kernel, dim3(Hq + 2 * Hkv, M), dim3(64), 0, (hipStream_t)stream, qkv, ldq, Hq, Hkv,
                     q_norm, k_norm, eps, pos0, theta, q_out, k_cache, vt_cache, maxlen);
  return skinny_check_launch("qk_rope_store");
}

extern "C" size_t skinny_attn_workspace_bytes(int Hkv, int maxlen) {
  const size_t nch = (size_t)((maxlen + kChunk - 1) / kChunk);
  return (size_t)Hkv * nch * kRowsMax * (kD + 2) * sizeof(float);
}

extern "C" int skinny_attention_bf16(const uint16_t* q, int M, int Hq, int Hkv, int D, const uint16_t* k_cache,
                                     const uint16_t* vt_cache, int maxlen, const int32_t* pos0, float scale,
                                     float* workspace, size_t workspace_bytes, uint16_t* out, void* stream) {
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
  hipLaunchKernelGGL(attn_chunk_kernel, dim3(nch, Hkv), dim3(64 * kWaves), 0, (hipStream_t)stream, q, M, Hq, Hkv,
                     k_cache, vt_cache, maxlen, pos0, scale, part_o, part_ml, nch);
  int rc = skinny_check_launch("attention");
  if (rc) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(Hq, M), dim3(64), 0, (hipStream_t)stream, part_o, part_ml, M, Hq, Hkv,
                     pos0, nch, out);
  return skinny_check_launch("attention combine");
}
