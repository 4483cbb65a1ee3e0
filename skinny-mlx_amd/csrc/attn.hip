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

#include "common.h"

namespace {

constexpr int kD = 128;             // head dim
constexpr int kWaves = 4;           // waves per workgroup: one 16-row tile each
constexpr int kChunk = 128;         // keys per workgroup
constexpr int kRowsMax = 64;        // GQA group (<= 4) x M (<= 16)

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

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
    const float ss = wave_sum(a * a + b * b);
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
    uint16_t* dst = kc + ((size_t)(head - Hq) * maxlen + slot) * kD;
    dst[lane] = ra;
    dst[lane + 64] = rb;
  }
}

// --- chunked attention ------------------------------------------------------------------------

// Draft-tree descriptor (NULL = causal): tree[0] = b, the tree's key slots are [pos0 - b,
// pos0 - b + 32); tree[1 + t] = bit mask over those slots of the keys token t sees there (its
// ancestors and itself); tree[1 + M + t] = token t's RoPE position relative to pos0. Keys before
// the tree are always visible, keys after it never. A chain (masks 2^(t+1) - 1, positions t,
// b = 0) is exactly the causal mask.

// LDS row pitch of the staged K rows and V^T rows (bf16): 128 values + 8 of padding, so the 16
// lanes that read one 16-byte column of 16 consecutive rows hit different banks.
constexpr int kPitch = kD + 8;
constexpr float kLog2e = 1.4426950408889634f;

// Workgroup (chunk c, kv head h), keys [128c, 128c + 128). The workgroup stages the chunk's K
// rows and V^T rows in LDS (each thread eight 16-byte loads of each); wave w takes the 16 query
// rows 16w .. 16w + 15 of the (token, group head) rows, at most 64 rows in all.
//
// Scores are computed transposed, S^T = K Q^T (K rows as the A operand, Q as B), with the 16 K
// rows of tile kt taken in the order row r -> key 32(kt/2) + 8(r/4) + 4(kt%2) + r%4. The
// accumulators then leave lane (col, quad) holding, for ONE query row (16w + col), the keys
// 32s + 8quad + 0..7 of every 32-key step s (tiles 2s and 2s+1): the row maximum and sum are
// the lane's own 32 values plus two shuffles across the quads, and the bf16 P is already the
// A operand of the P.V MFMA (slot 8quad + j = key 32s + 8quad + j, the V^T rows read as B) —
// no LDS round trip and no per-element index arithmetic. Exponents are base 2 (v_exp_f32) with
// log2(e) folded into the scale; the partial's row maximum is stored in those units.
// Chunk boundaries sit at fixed absolute key positions and every sum runs in a fixed order, so
// a row's partials never depend on how many rows share the step.
//
// Fused form (kFused): `q` is the raw q|k|v rows of the step (row stride fa.ldq) and the kernel
// does what skinny_qk_rope_store would have done first. Each lane normalises and rotates its own
// query row in the B-operand layout (the RMSNorm's sum of squares over the row's 128 dims is the
// lane's 32 plus two shuffles across the quads; the rotate-half pairs, dims d and d + 64, sit in
// the same lane), with cos/sin from a table built by the expressions the separate kernel
// evaluates. The workgroup whose chunk holds a new token's slot computes that token's key row
// exactly as the separate kernel does (one wave per token, lanes d and d + 64), writes key and
// value to the caches and into its own LDS copy of the chunk. One launch fewer per layer.
struct FusedArgs {
  int ldq;                 // row stride of the q|k|v rows
  const uint16_t* qn;      // q RMSNorm weight [128] or NULL
  const uint16_t* kn;      // k RMSNorm weight [128] or NULL
  float eps;
  const float* rope;       // [positions][64] (cos, sin)
};

constexpr int kFusedMaxTokens = 4 * kWaves;  // new tokens per step in the fused form (4 per wave)

template <bool kFused>
// The device position comes first among the arguments: it is the kernel's first read, and the
// leading argument dwords arrive preloaded in SGPRs.
__global__ __launch_bounds__(64 * kWaves) void attn_chunk_kernel(const int32_t* __restrict__ pos0,
                                                                 const uint16_t* __restrict__ q, FusedArgs fa, int M,
                                                                 int Hq, int Hkv, uint16_t* __restrict__ kc,
                                                                 uint16_t* __restrict__ vt, int maxlen, float scale,
                                                                 const int32_t* __restrict__ tree,
                                                                 float* __restrict__ part_o, float* __restrict__ part_ml,
                                                                 int nchunk_max) {
  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[kChunk * kPitch];  // K rows: [key][dim]
  __shared__ __attribute__((aligned(16))) uint16_t vs_lds[kD * kPitch];      // V^T rows: [dim][key]
  const int c = blockIdx.x, h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int p0 = pos0[0];
  const int total = p0 + M;  // keys present after this step's tokens were stored
  if (c * kChunk >= total) return;
  const int G = Hq / Hkv;
  const int rows = G * M;
  const int key0 = c * kChunk;
  const int col = lane & 15, quad = lane >> 4;
  const bool busy = wave * 16 < rows;

  // 1. Loads, in the order their data is needed: this lane's query row (the B operand, dims
  //    32ks + 8quad .. +8; fused: raw, with its norm weights and RoPE factors), the fused form's
  //    new key/value rows, then the chunk's K rows and V^T rows (16-byte pieces, 16 per row). The
  //    in-order load counter then lets the query work start while the chunk is still in flight.
  // Visibility of key kp for this lane's row, one formula for both masks: with j = kp - tbase,
  // visible iff j < 0, or j < 32 and bit j of tmask. Causal: tbase = p0 + t + 1, tmask = 0. Draft
  // tree: the tree's first slot and the token's mask. A padding row sees nothing (tbase = key0).
  const int qrow = wave * 16 + col;
  const bool live = busy && qrow < rows;
  const int t = live ? qrow / G : 0;
  bf16x8_t qf[4];
  u32x4_t raw[4], wq[4];
  f32x4_t cs[2][4];  // fused: (cos, sin) of dims 32ks + 8quad + e, e = 0..7, for ks = 0, 1
  int tbase = key0;
  uint32_t tmask = 0;
  if constexpr (kFused) {
    // Every lane loads (a lane without a row reads token 0's, and ignores it), and nothing loaded
    // here is used before the chunk's loads are issued below: a use, or a branch around a load,
    // would make the wave wait for these loads first.
    const int qg = live ? qrow % G : 0;
    const uint16_t* qr = q + (size_t)t * fa.ldq + ((size_t)h * G + qg) * kD;
    const int pos = p0 + (tree ? tree[1 + M + t] : t);
    const uint16_t* qn = fa.qn ? fa.qn : qr;  // no norm weight: the row itself, never used
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      raw[ks] = *reinterpret_cast<const u32x4_t*>(qr + ks * 32 + quad * 8);
      wq[ks] = *reinterpret_cast<const u32x4_t*>(qn + ks * 32 + quad * 8);
    }
    const f32x4_t* rp = reinterpret_cast<const f32x4_t*>(fa.rope + (size_t)pos * 128);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < 4; ++j) cs[ks][j] = rp[(ks * 32 + quad * 8) / 2 + j];
  }
  int tree0 = 0, tree_mask = 0;
  if (tree) {  // read by every lane (t = 0 without a row) and used after the chunk's loads
    tree0 = tree[0];
    tree_mask = tree[1 + t];
  }
  if (live) {
    if constexpr (!kFused) {
      const uint16_t* qr = q + ((size_t)t * Hq + h * G + qrow % G) * kD;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const bf16x8_t*>(qr + ks * 32 + quad * 8);
    }
  } else {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[ks] = bf16x8_t{};
  }
  // Fused: raw key (dims lane, lane + 64), value and RoPE factors of the new tokens whose slots
  // fall in this chunk (wave w: tokens w + 4i).
  int new_row[4];
  uint32_t nraw[4], nval[4], kw = 0;
  uint16_t nk0[4], nk1[4], nv0[4], nv1[4], kw0 = 0, kw1 = 0;  // combined after the chunk's loads
  float2 ncs[4];
  if constexpr (kFused) {
    const uint16_t* kn = fa.kn ? fa.kn : q;  // no norm weight: never used
    kw0 = kn[lane];
    kw1 = kn[lane + 64];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tt = wave + kWaves * i;
      const int slot = p0 + tt;
      const bool mine = tt < M && slot >= key0 && slot < key0 + kChunk;
      const int tl = mine ? tt : 0;  // otherwise token 0's rows are read and ignored
      new_row[i] = mine ? slot - key0 : -1;
      const uint16_t* src = q + (size_t)tl * fa.ldq + (size_t)(Hq + h) * kD;
      const uint16_t* vsrc = q + (size_t)tl * fa.ldq + (size_t)(Hq + Hkv + h) * kD;
      nk0[i] = src[lane];
      nk1[i] = src[lane + 64];
      nv0[i] = vsrc[lane];
      nv1[i] = vsrc[lane + 64];
      const int pos = p0 + (tree ? tree[1 + M + tl] : tl);
      ncs[i] = reinterpret_cast<const float2*>(fa.rope)[(size_t)pos * 64 + lane];
    }
  }
  const u32x4_t* kh = reinterpret_cast<const u32x4_t*>(kc + ((size_t)h * maxlen + key0) * kD);
  const uint16_t* vh = vt + (size_t)h * kD * maxlen + key0;
  u32x4_t kr[8], vr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = threadIdx.x + i * 64 * kWaves;  // piece e: row e / 16, column piece e % 16
    kr[i] = kh[e];
    vr[i] = *reinterpret_cast<const u32x4_t*>(vh + (size_t)(e >> 4) * maxlen + (e & 15) * 8);
  }
  if (live) {
    tbase = tree ? p0 - tree0 : p0 + t + 1;
    tmask = tree ? (uint32_t)tree_mask : 0u;
  }
  if constexpr (kFused) {
    if (fa.kn) kw = (uint32_t)kw0 | ((uint32_t)kw1 << 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool mine = new_row[i] >= 0;
      nraw[i] = mine ? (uint32_t)nk0[i] | ((uint32_t)nk1[i] << 16) : 0u;
      nval[i] = mine ? (uint32_t)nv0[i] | ((uint32_t)nv1[i] << 16) : 0u;
      if (!mine) ncs[i] = float2{1.f, 0.f};
    }
  }
  // Fused: the query row's RMSNorm (the lane's 32 squares plus two shuffles across the quads)
  // and RoPE (dims d and d + 64 in the same lane), into the B operand.
  if constexpr (kFused) {
    if (live) {
      float x[4][8];
      float ss = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[ks][e] = bf16_bits_to_f32((e & 1) ? (raw[ks][e >> 1] >> 16) : (raw[ks][e >> 1] & 0xffffu));
          ss = fmaf(x[ks][e], x[ks][e], ss);
        }
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      if (fa.qn) {
        const float inv = rsqrtf(ss / (float)kD + fa.eps);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float wv = bf16_bits_to_f32((e & 1) ? (wq[ks][e >> 1] >> 16) : (wq[ks][e >> 1] & 0xffffu));
            x[ks][e] = bf16_bits_to_f32(f32_to_bf16_bits(x[ks][e] * inv * wv));
          }
      }
      u32x4_t lo[2], hi[2];  // rotated dims 32ks + 8quad + e (lo) and those + 64 (hi)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          uint32_t wl = 0, wh = 0;
#pragma unroll
          for (int bb = 0; bb < 2; ++bb) {
            const int e = 2 * e2 + bb;
            const float c2 = cs[ks][e >> 1][(e & 1) * 2], sn = cs[ks][e >> 1][(e & 1) * 2 + 1];
            const float av = x[ks][e], bv = x[ks + 2][e];
            wl |= (uint32_t)f32_to_bf16_bits(av * c2 - bv * sn) << (16 * bb);
            wh |= (uint32_t)f32_to_bf16_bits(bv * c2 + av * sn) << (16 * bb);
          }
          lo[ks][e2] = wl;
          hi[ks][e2] = wh;
        }
      qf[0] = __builtin_bit_cast(bf16x8_t, lo[0]);
      qf[1] = __builtin_bit_cast(bf16x8_t, lo[1]);
      qf[2] = __builtin_bit_cast(bf16x8_t, hi[0]);
      qf[3] = __builtin_bit_cast(bf16x8_t, hi[1]);
    }
  }
  // Fused: the new key rows, exactly as skinny_qk_rope_store makes them (the same 64-lane sum of
  // the RMSNorm, for the wave's tokens side by side), into the caches.
  uint32_t new_k[4];
  if constexpr (kFused) {
    float ka[4], kb[4], ss[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ka[i] = bf16_bits_to_f32(nraw[i] & 0xffffu);
      kb[i] = bf16_bits_to_f32(nraw[i] >> 16);
      ss[i] = ka[i] * ka[i] + kb[i] * kb[i];
    }
    if (fa.kn) {
#pragma unroll
      for (int i = 0; i < 4; ++i) ss[i] = wave_sum(ss[i]);
      const float w0 = bf16_bits_to_f32(kw & 0xffffu), w1 = bf16_bits_to_f32(kw >> 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float inv = rsqrtf(ss[i] / (float)kD + fa.eps);
        ka[i] = bf16_bits_to_f32(f32_to_bf16_bits(ka[i] * inv * w0));
        kb[i] = bf16_bits_to_f32(f32_to_bf16_bits(kb[i] * inv * w1));
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t ra = f32_to_bf16_bits(ka[i] * ncs[i].x - kb[i] * ncs[i].y);
      const uint16_t rb = f32_to_bf16_bits(kb[i] * ncs[i].x + ka[i] * ncs[i].y);
      new_k[i] = (uint32_t)ra | ((uint32_t)rb << 16);
      if (new_row[i] < 0) continue;
      const int slot = key0 + new_row[i];
      uint16_t* kdst = kc + ((size_t)h * maxlen + slot) * kD;
      kdst[lane] = ra;
      kdst[lane + 64] = rb;
      vt[((size_t)h * kD + lane) * maxlen + slot] = (uint16_t)(nval[i] & 0xffffu);
      vt[((size_t)h * kD + lane + 64) * maxlen + slot] = (uint16_t)(nval[i] >> 16);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = threadIdx.x + i * 64 * kWaves;
    *reinterpret_cast<u32x4_t*>(&ks_lds[(e >> 4) * kPitch + (e & 15) * 8]) = kr[i];
    *reinterpret_cast<u32x4_t*>(&vs_lds[(e >> 4) * kPitch + (e & 15) * 8]) = vr[i];
  }
  __syncthreads();
  if constexpr (kFused) {  // the new rows replace whatever the staged slots held
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = new_row[i];
      if (r < 0) continue;
      ks_lds[r * kPitch + lane] = (uint16_t)(new_k[i] & 0xffffu);
      ks_lds[r * kPitch + lane + 64] = (uint16_t)(new_k[i] >> 16);
      vs_lds[lane * kPitch + r] = (uint16_t)(nval[i] & 0xffffu);
      vs_lds[(lane + 64) * kPitch + r] = (uint16_t)(nval[i] >> 16);
    }
    __syncthreads();
  }
  if (!busy) return;

  // 2. S^T tiles: element i of tile kt is the score of key 32(kt/2) + 8quad + 4(kt%2) + i.
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  float s[8][4];
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) {
    const int krow = 32 * (kt >> 1) + 8 * (col >> 2) + 4 * (kt & 1) + (col & 3);
    f32x4_t acc = zero;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      acc = mfma16x16x32(*reinterpret_cast<const bf16x8_t*>(&ks_lds[krow * kPitch + ks * 32 + quad * 8]), qf[ks], acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) s[kt][i] = acc[i];
  }

  // 3. Visibility, the row maximum (log2 units), bf16 P packed as the P.V A operand, its sum.
  const float sc = scale * kLog2e;
  const int kq = key0 + 8 * quad;  // key of element (kt, i) = kq + 32(kt/2) + 4(kt%2) + i
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 8; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = kq + 32 * (kt >> 1) + 4 * (kt & 1) + i - tbase;
      const uint32_t vis = (uint32_t)(j < 0) | ((uint32_t)(j < 32) & (tmask >> (j & 31)));
      s[kt][i] = (vis & 1u) ? s[kt][i] * sc : -INFINITY;
      mx = fmaxf(mx, s[kt][i]);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float mref = mx == -INFINITY ? 0.f : mx;  // a row with no visible key here: every P is 0
  u32x4_t pa[4];
  float sum = 0.f;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int w = 0; w < 4; ++w) {  // word w: elements 2(w%2), 2(w%2)+1 of tile 2ks + w/2
      const int kt = 2 * ks + (w >> 1), i = 2 * (w & 1);
      const uint16_t b0 = f32_to_bf16_bits(__builtin_amdgcn_exp2f(s[kt][i] - mref));
      const uint16_t b1 = f32_to_bf16_bits(__builtin_amdgcn_exp2f(s[kt][i + 1] - mref));
      sum += bf16_bits_to_f32(b0);
      sum += bf16_bits_to_f32(b1);
      pa[ks][w] = (uint32_t)b0 | ((uint32_t)b1 << 16);
    }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);

  // 4. O = P V over the 4 key steps of 32; lane holds O rows 4quad + i, dim 16dt + col.
  f32x4_t o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = zero;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, pa[ks]);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      o[dt] = mfma16x16x32(pf, *reinterpret_cast<const bf16x8_t*>(&vs_lds[(dt * 16 + col) * kPitch + ks * 32 + quad * 8]),
                           o[dt]);
  }

  // 5. The chunk partial of this wave's rows.
  const size_t base = ((size_t)h * nchunk_max + c) * kRowsMax + wave * 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float* dst = part_o + (base + quad * 4 + i) * kD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) dst[dt * 16 + col] = o[dt][i];
  }
  if (quad == 0) {
    part_ml[(base + col) * 2] = mx;
    part_ml[(base + col) * 2 + 1] = sum;
  }
}

// One wave per (q head, token): merge the chunk partials, normalise, store bf16. Chunks are taken
// in blocks of 32 by absolute index: all of a block's loads are issued together (lane c holds
// chunk c's statistics, every lane its two dims of every chunk's partial row), then the block is
// folded into running sums in chunk order, rescaled when the running maximum grows. A block past
// a row's position holds only empty chunks and rescales by exactly 1, so the result does not
// depend on how many tokens share the step.
constexpr int kCombineBlock = 32;

__global__ __launch_bounds__(64) void attn_combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                                          int M, int Hq, int Hkv, const int32_t* __restrict__ pos0,
                                                          int nchunk_max, uint16_t* __restrict__ out) {
  const int hq = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const int G = Hq / Hkv, h = hq / G, row = t * G + hq % G;
  const size_t head_base = (size_t)h * nchunk_max * kRowsMax + row;  // chunk c at + c * kRowsMax
  // The first block's partials are loaded before the chunk count is known (it needs *pos0):
  // every chunk the workspace holds up to kCombineBlock, the ones past the context discarded below
  // by selection (their stale values never enter an arithmetic operation).
  const int pre = min(kCombineBlock, nchunk_max);
  float mc_pre = -INFINITY, lc_pre = 0.f;
  float o0[kCombineBlock], o1[kCombineBlock];
  if (lane < pre) {
    mc_pre = part_ml[(head_base + (size_t)lane * kRowsMax) * 2];
    lc_pre = part_ml[(head_base + (size_t)lane * kRowsMax) * 2 + 1];
  }
#pragma unroll
  for (int j = 0; j < kCombineBlock; ++j) {
    o0[j] = o1[j] = 0.f;
    if (j < pre) {
      const float* po = part_o + (head_base + (size_t)j * kRowsMax) * kD;
      o0[j] = po[lane];
      o1[j] = po[lane + 64];
    }
  }
  const int total = pos0[0] + M;
  const int nch = (total + kChunk - 1) / kChunk;
  float run_m = -INFINITY, run_l = 0.f, a0 = 0.f, a1 = 0.f;
  for (int c0 = 0; c0 < nch; c0 += kCombineBlock) {
    const int nb = min(kCombineBlock, nch - c0);
    float mc = -INFINITY, lc = 0.f;
    if (c0 == 0) {
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
  const float inv = run_l > 0.f ? 1.0f / run_l : 0.f;
  uint16_t* dst = out + ((size_t)t * Hq + hq) * kD;
  dst[lane] = f32_to_bf16_bits(a0 * inv);
  dst[lane + 64] = f32_to_bf16_bits(a1 * inv);
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
  hipLaunchKernelGGL(attn_combine_kernel, dim3(Hq, M), dim3(64), 0, (hipStream_t)stream, part_o, part_ml, M, Hq, Hkv,
                     pos0, nch, out);
  return skinny_check_launch("attention combine");
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
  hipLaunchKernelGGL(attn_combine_kernel, dim3(Hq, M), dim3(64), 0, (hipStream_t)stream, part_o, part_ml, M, Hq, Hkv,
                     pos0, nch, out);
  return skinny_check_launch("attention combine");
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
