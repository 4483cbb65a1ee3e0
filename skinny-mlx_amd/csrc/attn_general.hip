// Full attention of the verify step for head layouts the tuned 128-dim kernels (attn.hip) do not
// take: head_dim 64, 128 or 256, RoPE over only the first R dims of each head, query heads laid out
// with a stride (Qwen3.5's q_proj holds per head the query rows then the gate rows), and the
// attention output gated by sigmoid(gate) before o_proj.
//
// Reference behaviour: the full-attention layers of mlx_lm's Qwen3.5 decoder that the reference
// loads (skinny_mlx/spec.py:175, mlx-community/Qwen3.5-4B-MLX-4bit) and runs at spec.py:24-29 —
// per-head q/k RMSNorm, rotate-half RoPE over a quarter of each 256-dim head, causal GQA attention,
// output * sigmoid(gate) (transformers qwen3_5 Attention forward states the same arithmetic).
//
// Three launches per call: (1) q/k RMSNorm + partial RoPE, the query rows to a workspace, the new
// keys and values into the caches; (2) one workgroup per (chunk, kv head), the chunk's K and V^T
// rows staged in LDS, its scores and P.V on MFMA; (3) one workgroup per (query head, token)
// merging the chunks in chunk order, then the gate. Every row depends only on its own data and
// every sum runs in a fixed order over absolute key positions, so a token's output does not depend
// on how many tokens share the step. Cache layout as attn.hip: K [Hkv][maxlen][D], V^T
// [Hkv][D][maxlen]; the cached length is read from device memory.
#include "common.h"

namespace {

constexpr int kGWaves = 4;      // waves per chunk workgroup: one 16-row tile each
constexpr int kGChunk = 128;    // keys per chunk workgroup for 64- and 128-dim heads; maxlen's granule
constexpr int kGRowsMax = 64;   // GQA group x tokens per kv head
constexpr int kGMaxTokens = 16; // tokens per call (the query rows' workspace)
constexpr float kGLog2e = 1.4426950408889634f;
constexpr int kGCombineBlock = 64;  // chunks the merge loads at once (lane j: chunk c0 + j)

// Keys per chunk workgroup: 64 for 256-dim heads, so that a chunk's K and V^T rows (32 KB each)
// fit in LDS twice per CU and a 2048-key context gives 32 chunks per kv head.
__host__ __device__ constexpr int general_chunk(int D) { return D == 256 ? 64 : kGChunk; }

// Workspace: the normalised, rotated query rows, then the chunk partials (fp32 O rows, then the
// row maximum in log2 units and the row sum).
struct GeneralLayout {
  size_t q, o, ml, bytes;
  __host__ __device__ GeneralLayout(int Hq, int Hkv, int D, int nch) {
    q = 0;
    o = ((size_t)kGMaxTokens * Hq * D * 2 + 255) & ~(size_t)255;
    ml = o + (size_t)Hkv * nch * kGRowsMax * D * 4;
    bytes = ml + (size_t)Hkv * nch * kGRowsMax * 2 * 4;
  }
};

// Where the heads sit in a q|k|v row: query head h at h * qs, key head j at koff + j * D, value
// head j at voff + j * D, and (gated layers) the gate of query head h at goff + h * qs.
struct HeadLayout {
  int ldq, qs, koff, voff, goff;
};

// (1) One wave per (head, token): heads [0, Hq) are queries, [Hq, Hq + Hkv) keys, then values.
// Lane l holds dims l + 64e. The RMSNorm is the wave sum of the squares; each normalised value is
// rounded to bf16, then the first R dims turn as pairs (i, i + R/2) with the (cos, sin) of
// table[pos][i] and are rounded again (the order of attn.hip's qk_rope_store_kernel).
template <int D>
__global__ __launch_bounds__(64) void general_qk_store_kernel(const int32_t* __restrict__ pos0,
                                                              const uint16_t* __restrict__ qkv, HeadLayout hl, int Hq,
                                                              int Hkv, const uint16_t* __restrict__ qn,
                                                              const uint16_t* __restrict__ kn, float eps, int R,
                                                              const float* __restrict__ rope,
                                                              const int32_t* __restrict__ tree, int M,
                                                              uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                                              uint16_t* __restrict__ vt, int maxlen) {
  constexpr int E = D / 64;
  __shared__ float row[D];
  const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const int p0 = pos0[0];
  const int slot = p0 + t;
  const int pos = p0 + (tree ? tree[1 + M + t] : t);
  const uint16_t* src;
  if (head < Hq) src = qkv + (size_t)t * hl.ldq + (size_t)head * hl.qs;
  else if (head < Hq + Hkv) src = qkv + (size_t)t * hl.ldq + hl.koff + (size_t)(head - Hq) * D;
  else src = qkv + (size_t)t * hl.ldq + hl.voff + (size_t)(head - Hq - Hkv) * D;
  uint16_t raw[E];
#pragma unroll
  for (int e = 0; e < E; ++e) raw[e] = src[lane + 64 * e];
  if (head >= Hq + Hkv) {  // value: into the transposed cache as it is
    const int h = head - Hq - Hkv;
#pragma unroll
    for (int e = 0; e < E; ++e) vt[((size_t)h * D + lane + 64 * e) * maxlen + slot] = raw[e];
    return;
  }
  float x[E];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    x[e] = bf16_bits_to_f32(raw[e]);
    ss = fmaf(x[e], x[e], ss);
  }
  const uint16_t* nw = head < Hq ? qn : kn;
  if (nw) {
    const float inv = rsqrtf(wave_sum(ss) / (float)D + eps);
#pragma unroll
    for (int e = 0; e < E; ++e)
      x[e] = bf16_bits_to_f32(f32_to_bf16_bits(x[e] * inv * bf16_bits_to_f32(nw[lane + 64 * e])));
  }
#pragma unroll
  for (int e = 0; e < E; ++e) row[lane + 64 * e] = x[e];
  __syncthreads();
  const int half = R >> 1;
  uint16_t outv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int d = lane + 64 * e;
    if (d < R) {
      const int i = d < half ? d : d - half;
      const float a = row[i], b = row[i + half];
      const float c = rope[((size_t)pos * half + i) * 2], s = rope[((size_t)pos * half + i) * 2 + 1];
      outv[e] = f32_to_bf16_bits(d < half ? a * c - b * s : b * c + a * s);
    } else {
      outv[e] = f32_to_bf16_bits(x[e]);
    }
  }
  uint16_t* dst = head < Hq ? q_out + ((size_t)t * Hq + head) * D : kc + ((size_t)(head - Hq) * maxlen + slot) * D;
#pragma unroll
  for (int e = 0; e < E; ++e) dst[lane + 64 * e] = outv[e];
}

// (2) Workgroup (chunk c, kv head h), keys [CH c, CH c + CH); wave w takes the query rows
// 16w .. 16w + 15 of the (token, group head) rows. attn.hip's chunk kernel over D dims: every thread
// issues its 16-byte pieces of the chunk's K rows and V^T rows at once (PIECES of each), they go to
// LDS (pitches D + 8 and CH + 8: the 16 rows one 16-byte read spans fall on distinct banks), and the
// busy waves compute S^T = K Q^T with the K rows of tile kt taken in the order row r -> key
// 32(kt/2) + 8(r/4) + 4(kt%2) + r%4, so that lane (col, quad) holds the keys 32s + 8quad + 0..7 of
// its query row and its bf16 P is the A operand of P.V; base-2 exponents with log2(e) in the scale.
template <int D>
__global__ __launch_bounds__(64 * kGWaves) void general_chunk_kernel(const int32_t* __restrict__ pos0,
                                                                     const uint16_t* __restrict__ q, int M, int Hq,
                                                                     int Hkv, const uint16_t* __restrict__ kc,
                                                                     const uint16_t* __restrict__ vt, int maxlen,
                                                                     float scale, const int32_t* __restrict__ tree,
                                                                     float* __restrict__ part_o,
                                                                     float* __restrict__ part_ml, int nchunk_max) {
  constexpr int CH = general_chunk(D);
  constexpr int KS = D / 32;   // 32-dim steps of a score
  constexpr int DT = D / 16;   // 16-dim tiles of an output row
  constexpr int KT = CH / 16;  // 16-key tiles of the chunk
  constexpr int PS = CH / 32;  // 32-key steps of P.V
  constexpr int KP = D + 8, VP = CH + 8;
  constexpr int PIECES = CH * D / 8 / (64 * kGWaves);  // 16-byte pieces per thread of K, and of V^T
  static_assert(PIECES * 8 * 64 * kGWaves == CH * D, "the chunk splits evenly over the threads");
  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[CH * KP];  // K rows: [key][dim]
  __shared__ __attribute__((aligned(16))) uint16_t vs_lds[D * VP];   // V^T rows: [dim][key]
  const int c = blockIdx.x, h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int p0 = pos0[0];
  const int total = p0 + M;
  const int key0 = c * CH;
  if (key0 >= total) return;
  const int G = Hq / Hkv;
  const int rows = G * M;
  const bool busy = wave * 16 < rows;
  const int col = lane & 15, quad = lane >> 4;
  const int qrow = wave * 16 + col;
  const bool live = busy && qrow < rows;
  const int t = live ? qrow / G : 0;
  // Loads in the order their data is needed: the query row (B operand), the tree words, the chunk.
  bf16x8_t qf[KS];
  if (live) {
    const uint16_t* qr = q + ((size_t)t * Hq + h * G + qrow % G) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = *reinterpret_cast<const bf16x8_t*>(qr + ks * 32 + quad * 8);
  } else {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = bf16x8_t{};
  }
  int tree0 = 0, tree_mask = 0;
  if (tree) {
    tree0 = tree[0];
    tree_mask = tree[1 + t];
  }
  const u32x4_t* kh = reinterpret_cast<const u32x4_t*>(kc + ((size_t)h * maxlen + key0) * D);
  const uint16_t* vh = vt + (size_t)h * D * maxlen + key0;
  u32x4_t kr[PIECES], vr[PIECES];
#pragma unroll
  for (int i = 0; i < PIECES; ++i) {
    const int e = threadIdx.x + i * 64 * kGWaves;  // K piece e: row e / (D/8); V^T piece e: row e / (CH/8)
    kr[i] = kh[e];
    vr[i] = *reinterpret_cast<const u32x4_t*>(vh + (size_t)(e / (CH / 8)) * maxlen + (e % (CH / 8)) * 8);
  }
  // Visibility of key kp for this lane's row: with j = kp - tbase, visible iff j < 0, or j < 32
  // and bit j of tmask. Causal: tbase = p0 + t + 1, tmask = 0; a draft tree: the tree's first slot
  // and the token's ancestor mask; a padding row sees nothing.
  int tbase = key0;
  uint32_t tmask = 0;
  if (live) {
    tbase = tree ? p0 - tree0 : p0 + t + 1;
    tmask = tree ? (uint32_t)tree_mask : 0u;
  }
#pragma unroll
  for (int i = 0; i < PIECES; ++i) {
    const int e = threadIdx.x + i * 64 * kGWaves;
    *reinterpret_cast<u32x4_t*>(&ks_lds[(e / (D / 8)) * KP + (e % (D / 8)) * 8]) = kr[i];
    *reinterpret_cast<u32x4_t*>(&vs_lds[(e / (CH / 8)) * VP + (e % (CH / 8)) * 8]) = vr[i];
  }
  __syncthreads();
  if (!busy) return;

  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  float s[KT][4];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const int krow = 32 * (kt >> 1) + 8 * (col >> 2) + 4 * (kt & 1) + (col & 3);
    f32x4_t acc = zero;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      acc = mfma16x16x32(*reinterpret_cast<const bf16x8_t*>(&ks_lds[krow * KP + ks * 32 + quad * 8]), qf[ks], acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) s[kt][i] = acc[i];
  }
  const float sc = scale * kGLog2e;
  const int kq = key0 + 8 * quad;
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = kq + 32 * (kt >> 1) + 4 * (kt & 1) + i - tbase;
      const uint32_t vis = (uint32_t)(j < 0) | ((uint32_t)(j < 32) & (tmask >> (j & 31)));
      s[kt][i] = (vis & 1u) ? s[kt][i] * sc : -INFINITY;
      mx = fmaxf(mx, s[kt][i]);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float mref = mx == -INFINITY ? 0.f : mx;
  u32x4_t pa[PS];
  float sum = 0.f;
#pragma unroll
  for (int ks = 0; ks < PS; ++ks)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int kt = 2 * ks + (w >> 1), i = 2 * (w & 1);
      const uint16_t b0 = f32_to_bf16_bits(__builtin_amdgcn_exp2f(s[kt][i] - mref));
      const uint16_t b1 = f32_to_bf16_bits(__builtin_amdgcn_exp2f(s[kt][i + 1] - mref));
      sum += bf16_bits_to_f32(b0);
      sum += bf16_bits_to_f32(b1);
      pa[ks][w] = (uint32_t)b0 | ((uint32_t)b1 << 16);
    }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  // O = P V: lane holds O rows 4quad + i, dim 16dt + col; V^T row (16dt + col) keys 32ks + 8quad.
  f32x4_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = zero;
#pragma unroll
  for (int ks = 0; ks < PS; ++ks) {
    const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, pa[ks]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      o[dt] = mfma16x16x32(pf, *reinterpret_cast<const bf16x8_t*>(&vs_lds[(dt * 16 + col) * VP + ks * 32 + quad * 8]),
                           o[dt]);
  }
  const size_t base = ((size_t)h * nchunk_max + c) * kGRowsMax + wave * 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float* dst = part_o + (base + quad * 4 + i) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) dst[dt * 16 + col] = o[dt][i];
  }
  if (quad == 0) {
    part_ml[(base + col) * 2] = mx;
    part_ml[(base + col) * 2 + 1] = sum;
  }
}

// (3) One workgroup per (query head, token), max(1, D / 128) waves, lane l of wave w holding dims
// CW (w 64 + l) .. + CW - 1 (CW = D / 64 / waves, one 4- or 8-byte load per chunk): the merge of
// attn.hip's attn_combine_kernel. The chunk count comes first; then chunks are taken in blocks of
// kGCombineBlock by absolute index, lane j holding chunk c0 + j's statistics, a block's partial rows
// loaded in groups of 8 chunks, a group only when the block reaches into it (indices past the block's
// end repeat its last chunk), all before the first is used; the block is folded into running sums
// in chunk order, rescaled when the running maximum grows, the weights broadcast by v_readlane.
// With a gate, out = bf16(bf16(o) * bf16(sigmoid(gate))).
template <int D>
constexpr int general_combine_waves() { return D > 128 ? D / 128 : 1; }

template <int D>
__global__ __launch_bounds__(64 * general_combine_waves<D>()) void general_combine_kernel(
    const int32_t* __restrict__ pos0, const float* __restrict__ part_o, const float* __restrict__ part_ml, int M,
    int Hq, int Hkv, int nchunk_max, const uint16_t* __restrict__ qkv, HeadLayout hl, uint16_t* __restrict__ out) {
  constexpr int CH = general_chunk(D);
  constexpr int B = kGCombineBlock, GR = 8;
  constexpr int CW = D / 64 / general_combine_waves<D>();  // dims per lane: 1 or 2
  typedef __attribute__((ext_vector_type(CW))) float dims_t;
  const int hq = blockIdx.x, t = blockIdx.y, lane = threadIdx.x & 63;
  const int d0 = (int)threadIdx.x * CW;  // this lane's first dim
  const int G = Hq / Hkv, h = hq / G, row = t * G + hq % G;
  const size_t head_base = (size_t)h * nchunk_max * kGRowsMax + row;  // chunk c at + c * kGRowsMax
  const int nch = min((pos0[0] + M + CH - 1) / CH, nchunk_max);
  float run_m = -INFINITY, run_l = 0.f, a[CW];
#pragma unroll
  for (int k = 0; k < CW; ++k) a[k] = 0.f;
  for (int c0 = 0; c0 < nch; c0 += B) {
    const int nb = min(B, nch - c0);
    const size_t es = head_base + (size_t)(c0 + min(lane, nb - 1)) * kGRowsMax;
    float mc = part_ml[es * 2], lc = part_ml[es * 2 + 1];
    dims_t o[B];
#pragma unroll
    for (int g = 0; g < B / GR; ++g) {
      if (g * GR < nb) {
#pragma unroll
        for (int j = g * GR; j < (g + 1) * GR; ++j)
          o[j] = *reinterpret_cast<const dims_t*>(part_o + (head_base + (size_t)(c0 + min(j, nb - 1)) * kGRowsMax) * D + d0);
      }
    }
    mc = lane < nb ? mc : -INFINITY;
    lc = lane < nb ? lc : 0.f;
    float bm = mc;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) bm = fmaxf(bm, __shfl_xor(bm, off, 64));
    const float new_m = fmaxf(run_m, bm);
    const float keep = run_m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(run_m - new_m);
    run_l *= keep;
#pragma unroll
    for (int k = 0; k < CW; ++k) a[k] *= keep;
    const float wgt = mc == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc - new_m);
#pragma unroll
    for (int j = 0; j < B; ++j) {
      if (j < nb) {
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), j));
        run_l = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(lc), j)), wj, run_l);
#pragma unroll
        for (int k = 0; k < CW; ++k) a[k] = fmaf(o[j][k], wj, a[k]);
      }
    }
    run_m = new_m;
  }
  const float inv = run_l > 0.f ? 1.0f / run_l : 0.f;
  uint16_t* dst = out + ((size_t)t * Hq + hq) * D + d0;
#pragma unroll
  for (int k = 0; k < CW; ++k) {
    const uint16_t ob = f32_to_bf16_bits(a[k] * inv);
    if (hl.goff >= 0) {
      const float g = bf16_bits_to_f32(qkv[(size_t)t * hl.ldq + hl.goff + (size_t)hq * hl.qs + d0 + k]);
      const float sg = bf16_bits_to_f32(f32_to_bf16_bits(1.0f / (1.0f + expf(-g))));
      dst[k] = f32_to_bf16_bits(bf16_bits_to_f32(ob) * sg);
    } else {
      dst[k] = ob;
    }
  }
}

// cos/sin table of a RoPE over R dims: table[pos][i] = (cos, sin)(pos * theta^(-2i/R)), i < R/2,
// by the same expressions as attn.hip's table.
__global__ void rope_table_dim_kernel(float theta, int R, int positions, float* __restrict__ table) {
  const int half = R >> 1;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= positions * half) return;
  const int pos = idx / half, i = idx % half;
  const float inv_freq = powf(theta, -2.0f * (float)i / (float)R);
  float sn, cs;
  sincosf((float)pos * inv_freq, &sn, &cs);
  table[2 * idx] = cs;
  table[2 * idx + 1] = sn;
}

template <int D>
int launch_general(const int32_t* pos0, const uint16_t* qkv, const HeadLayout& hl, int M, int Hq, int Hkv,
                   const uint16_t* qn, const uint16_t* kn, float eps, int R, const float* rope,
                   const int32_t* tree, uint16_t* kc, uint16_t* vt, int maxlen, float scale, char* ws, int nch,
                   uint16_t* out, hipStream_t stream) {
  const GeneralLayout ly(Hq, Hkv, D, nch);
  uint16_t* q = reinterpret_cast<uint16_t*>(ws + ly.q);
  float* part_o = reinterpret_cast<float*>(ws + ly.o);
  float* part_ml = reinterpret_cast<float*>(ws + ly.ml);
  hipLaunchKernelGGL(general_qk_store_kernel<D>, dim3(Hq + 2 * Hkv, M), dim3(64), 0, stream, pos0, qkv, hl, Hq, Hkv, qn,
                     kn, eps, R, rope, tree, M, q, kc, vt, maxlen);
  if (int rc = skinny_check_launch("attention_general q/k")) return rc;
  hipLaunchKernelGGL(general_chunk_kernel<D>, dim3(nch, Hkv), dim3(64 * kGWaves), 0, stream, pos0, q, M, Hq, Hkv, kc,
                     vt, maxlen, scale, tree, part_o, part_ml, nch);
  if (int rc = skinny_check_launch("attention_general chunks")) return rc;
  hipLaunchKernelGGL(general_combine_kernel<D>, dim3(Hq, M), dim3(64 * general_combine_waves<D>()), 0, stream, pos0,
                     part_o, part_ml, M, Hq, Hkv, nch, qkv, hl, out);
  return skinny_check_launch("attention_general merge");
}

}  // namespace

extern "C" size_t skinny_attn_general_workspace_bytes(int Hq, int Hkv, int D, int maxlen) {
  if (Hq < 1 || Hkv < 1 || D < 1 || maxlen < 1) return 0;
  const int ch = general_chunk(D);
  return GeneralLayout(Hq, Hkv, D, (maxlen + ch - 1) / ch).bytes;
}

extern "C" int skinny_rope_table_dim(float theta, int rotary_dim, int positions, float* table, void* stream) {
  SKINNY_CHECK_ARG(table && positions >= 1 && theta > 1.f, "rope_table_dim: bad arguments");
  SKINNY_CHECK_ARG(rotary_dim >= 2 && rotary_dim % 2 == 0 && rotary_dim <= 256,
                   "rope_table_dim: rotary_dim=%d must be even, in [2, 256]", rotary_dim);
  const int n = positions * (rotary_dim / 2);
  hipLaunchKernelGGL(rope_table_dim_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, theta, rotary_dim,
                     positions, table);
  return skinny_check_launch("rope_table_dim");
}

extern "C" int skinny_attention_general_bf16(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D,
                                             int q_stride, int k_offset, int v_offset, int gate_offset,
                                             const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                             int rotary_dim, const float* rope_table, int rope_positions,
                                             const int32_t* pos0, const int32_t* tree, uint16_t* k_cache,
                                             uint16_t* vt_cache, int maxlen, float scale, void* workspace,
                                             size_t workspace_bytes, uint16_t* out, void* stream) {
  SKINNY_CHECK_ARG(qkv && rope_table && pos0 && k_cache && vt_cache && workspace && out,
                   "attention_general: null pointer");
  SKINNY_CHECK_ARG(D == 64 || D == 128 || D == 256, "attention_general: head dim %d unsupported (64, 128 or 256)", D);
  SKINNY_CHECK_ARG(Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "attention_general: Hq=%d not a multiple of Hkv=%d", Hq,
                   Hkv);
  SKINNY_CHECK_ARG(M >= 1 && M <= kGMaxTokens && (Hq / Hkv) * M <= kGRowsMax,
                   "attention_general: M=%d (at most %d) with %d query rows per kv head (at most %d)", M, kGMaxTokens,
                   (Hq / Hkv) * M, kGRowsMax);
  SKINNY_CHECK_ARG(rotary_dim >= 2 && rotary_dim % 2 == 0 && rotary_dim <= D,
                   "attention_general: rotary_dim=%d must be even, in [2, D=%d]", rotary_dim, D);
  SKINNY_CHECK_ARG(q_stride >= D && (gate_offset < 0 || gate_offset + (size_t)(Hq - 1) * q_stride + D <= (size_t)ldq),
                   "attention_general: q_stride=%d / gate_offset=%d do not fit the row of %d", q_stride, gate_offset,
                   ldq);
  SKINNY_CHECK_ARG(k_offset >= 0 && v_offset >= 0 && (size_t)(Hq - 1) * q_stride + D <= (size_t)ldq &&
                       (size_t)k_offset + (size_t)Hkv * D <= (size_t)ldq && (size_t)v_offset + (size_t)Hkv * D <= (size_t)ldq,
                   "attention_general: heads do not fit the q|k|v row of %d", ldq);
  SKINNY_CHECK_ARG(maxlen >= kGChunk && maxlen % kGChunk == 0 && rope_positions >= maxlen,
                   "attention_general: maxlen=%d must be a multiple of %d and within the RoPE table (%d)", maxlen,
                   kGChunk, rope_positions);
  SKINNY_CHECK_ARG(!tree || M <= 32, "attention_general: a draft tree holds at most 32 tokens (M=%d)", M);
  const int nch = maxlen / general_chunk(D);
  SKINNY_CHECK_ARG(workspace_bytes >= GeneralLayout(Hq, Hkv, D, nch).bytes,
                   "attention_general: workspace of %zu bytes, needs %zu", workspace_bytes,
                   GeneralLayout(Hq, Hkv, D, nch).bytes);
  SKINNY_CHECK_ARG(skinny_aligned(k_cache, 16) && skinny_aligned(vt_cache, 16) && skinny_aligned(workspace, 256) &&
                       skinny_aligned(qkv, 2) && skinny_aligned(rope_table, 8),
                   "attention_general: misaligned buffer");
  const HeadLayout hl{ldq, q_stride, k_offset, v_offset, gate_offset};
  char* ws = static_cast<char*>(workspace);
  const hipStream_t s = (hipStream_t)stream;
  switch (D) {
    case 64:
      return launch_general<64>(pos0, qkv, hl, M, Hq, Hkv, q_norm, k_norm, eps, rotary_dim, rope_table, tree, k_cache,
                                vt_cache, maxlen, scale, ws, nch, out, s);
    case 128:
      return launch_general<128>(pos0, qkv, hl, M, Hq, Hkv, q_norm, k_norm, eps, rotary_dim, rope_table, tree, k_cache,
                                 vt_cache, maxlen, scale, ws, nch, out, s);
    default:
      return launch_general<256>(pos0, qkv, hl, M, Hq, Hkv, q_norm, k_norm, eps, rotary_dim, rope_table, tree, k_cache,
                                 vt_cache, maxlen, scale, ws, nch, out, s);
  }
}
