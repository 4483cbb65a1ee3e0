// The chunk stage of the verify step's attention, shared by attn.hip (its kernels) and qmm.hip
// (the q|k|v projection fused with it): constants, the fused form's arguments, and the
// per-workgroup body. Internal to libskinny_hip.so.
#pragma once

#include "common.h"

namespace {

constexpr int kD = 128;             // head dim
constexpr int kWaves = 4;           // waves per workgroup: one 16-row tile each
constexpr int kChunk = 128;         // keys per workgroup
constexpr int kRowsMax = 64;        // GQA group (<= 4) x M (<= 16)

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
constexpr int kHandoffPolls = 1 << 14;       // polls (each a device-coherent round trip) before the wait form gives up

// The body of the chunk kernel for workgroup (chunk c, kv head h), shared by attn_chunk_kernel and
// the q|k|v projection + attention kernel of qmm.hip (kWait: see there).
template <bool kFused, bool kWait = false>
__device__ __forceinline__ void attn_chunk_body(int c, int h, const int32_t* __restrict__ pos0,
                                                const uint16_t* __restrict__ q, FusedArgs fa, int M, int Hq, int Hkv,
                                                uint16_t* __restrict__ kc, uint16_t* __restrict__ vt, int maxlen,
                                                float scale, const int32_t* __restrict__ tree,
                                                float* __restrict__ part_o, float* __restrict__ part_ml,
                                                int nchunk_max) {
  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[kChunk * kPitch];  // K rows: [key][dim]
  __shared__ __attribute__((aligned(16))) uint16_t vs_lds[kD * kPitch];      // V^T rows: [dim][key]
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
  const uint16_t* qr = q;  // fused: this lane's raw query row
  if constexpr (kFused) {
    // Every lane loads (a lane without a row reads token 0's, and ignores it), and nothing loaded
    // here is used before the chunk's loads are issued below: a use, or a branch around a load,
    // would make the wave wait for these loads first. kWait: the rows are loaded after the chunk.
    const int qg = live ? qrow % G : 0;
    qr = q + (size_t)t * fa.ldq + ((size_t)h * G + qg) * kD;
    const int pos = p0 + (tree ? tree[1 + M + t] : t);
    const uint16_t* qn = fa.qn ? fa.qn : qr;  // no norm weight: the row itself, never used
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if constexpr (!kWait) raw[ks] = *reinterpret_cast<const u32x4_t*>(qr + ks * 32 + quad * 8);
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
  const uint16_t* ksrc[4];
  const uint16_t* vsrc[4];
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
      ksrc[i] = q + (size_t)tl * fa.ldq + (size_t)(Hq + h) * kD;
      vsrc[i] = q + (size_t)tl * fa.ldq + (size_t)(Hq + Hkv + h) * kD;
      if constexpr (!kWait) {
        nk0[i] = ksrc[i][lane];
        nk1[i] = ksrc[i][lane + 64];
        nv0[i] = vsrc[i][lane];
        nv1[i] = vsrc[i][lane + 64];
      }
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
  if constexpr (kWait) {
    // The q|k|v rows come from the projection workgroups of the same launch, which publish them
    // with device-coherent stores into a buffer whose 16-bit words hold 0xFFFF (a NaN no rounded
    // sum takes) until written. Each lane reads its values with device-coherent loads and the
    // wave polls until none of them is still 0xFFFF; a bounded poll proceeds anyway, so a
    // missing value ends in wrong numbers, never a hang.
    static_assert(kFused, "the wait form reads the fused form's raw rows");
    auto ld32 = [](const uint16_t* p) {
      return __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto ld16 = [](const uint16_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto load_rows = [&]() {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int j = 0; j < 4; ++j) raw[ks][j] = ld32(qr + ks * 32 + quad * 8 + 2 * j);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        nk0[i] = ld16(ksrc[i] + lane);
        nk1[i] = ld16(ksrc[i] + lane + 64);
        nv0[i] = ld16(vsrc[i] + lane);
        nv1[i] = ld16(vsrc[i] + lane + 64);
      }
    };
    auto pending = [&]() {
      bool p = false;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int j = 0; j < 4; ++j) p |= (raw[ks][j] & 0xffffu) == 0xffffu || (raw[ks][j] >> 16) == 0xffffu;
#pragma unroll
      for (int i = 0; i < 4; ++i) p |= nk0[i] == 0xffffu || nk1[i] == 0xffffu || nv0[i] == 0xffffu || nv1[i] == 0xffffu;
      return p;
    };
    load_rows();
    for (int polls = 0; polls < kHandoffPolls; ++polls) {
      const bool mine = pending();
      if (__builtin_amdgcn_ballot_w64(mine) == 0) break;
      __builtin_amdgcn_s_sleep(2);
      if (mine) load_rows();
    }
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
            wl |= (uint32_t)f32_to_bf16_bits(fmaf(av, c2, -(bv * sn))) << (16 * bb);
            wh |= (uint32_t)f32_to_bf16_bits(fmaf(bv, c2, av * sn)) << (16 * bb);
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
  // the RMSNorm, for the wave's tokens side by side, and the same explicit fused multiply-adds, so
  // that no contraction the compiler chooses can round the two differently), into the caches.
  uint32_t new_k[4];
  if constexpr (kFused) {
    float ka[4], kb[4], ss[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ka[i] = bf16_bits_to_f32(nraw[i] & 0xffffu);
      kb[i] = bf16_bits_to_f32(nraw[i] >> 16);
      ss[i] = fmaf(kb[i], kb[i], ka[i] * ka[i]);
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
      const uint16_t ra = f32_to_bf16_bits(fmaf(ka[i], ncs[i].x, -(kb[i] * ncs[i].y)));
      const uint16_t rb = f32_to_bf16_bits(fmaf(kb[i], ncs[i].x, ka[i] * ncs[i].y));
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

}  // namespace

// The chunk-merge launch of attn.hip (attn_combine_kernel over (Hq, M) waves). With `reset`, the
// waves also put every 32-bit word of rows 0..M-1 of that buffer (reset_words words per row, row
// stride reset_ld words) back to 0xFFFFFFFF with device-coherent stores, for the q|k|v hand-off
// buffer of skinny_qkv_attention_fused_bf16.
int attn_combine_launch(const float* part_o, const float* part_ml, int M, int Hq, int Hkv, const int32_t* pos0,
                        int nchunk_max, uint16_t* out, uint32_t* reset, int reset_ld, int reset_words,
                        hipStream_t stream);
