// W4A16 affine group-64 "skinny" quantized matmul for 1..16 tokens on gfx950,
// and the load-time nibble relayout it reads.
//
// Reference behaviour: skinny_mlx/qmm.py:21-152 (Metal kernel skinny_qmm_4bit,
// repack_for_skinny, skinny_qmm). The arithmetic identity is the reference's
// (qmm.py:8-9): sum_k x (q s + b) = s * sum_k x q + b * sum_k x, applied once
// per 64-group. Everything else here is laid out for CDNA4:
//
//  * MFMA v_mfma_f32_16x16x32_bf16, tokens as the 16 A-rows (padded with zero
//    rows past M), 16 weight rows as the B-columns, 32 k per instruction, two
//    instructions per 64-group.
//  * Nibbles are fed to the MFMA raw: v_perm_b32 joins a code byte with a 0x43 byte
//    into bf16 128+q (exact), so the group result is
//      s * (G - 128*xs) + b * xs  =  s * G + (b - 128 s) * xs,
//    with G = sum x (128+q) and xs = sum x, both from MFMA (xs against a ones
//    operand, which lands directly in the accumulator lane layout).
//  * Weights are packed once into fragment order (skinny_w4g64_pack): per
//    (16-row tile, group pair) a 1152-byte block of 1 KB nibbles — 16 bytes per
//    lane, exactly its four B operands — followed by the 16 rows' scales and
//    biases for the two groups, so one wave stage is two contiguous loads.
//  * All loads are buffer loads against per-workgroup descriptors: the stage
//    offset is wave-uniform (SGPR) and the lane part constant. X rows past M use an
//    out-of-range offset and read as zeros without touching memory.
//
//  * Every wave owns RF row tiles x a contiguous range of group pairs and loads its own X
//    fragments (L2 hits); the `waves` waves of a workgroup split K and are reduced through
//    LDS in wave order. RF tiles share each X fragment, so RF trades X traffic against
//    workgroup count. (Splitting K across workgroups was measured and rejected on MI355X:
//    the agent-scope release each workgroup needs to publish its partial sums writes back
//    the XCD's L2, about 1 us each, serialised per XCD.)
//
// The tile depends on (K, N) only and every sum runs in a fixed order, so a token's output
// is bitwise identical for every M and every run.
#include <mutex>

#include "attn_chunk.h"

namespace {

// One MLX word (elements e0..e7 at bits 4e) -> fragment word: byte b holds e_b in its low
// nibble and e_{b+4} in its high nibble, so `& 0x0F0F0F0F` and `(>> 4) & 0x0F0F0F0F` leave
// one code per byte, ready for v_perm_b32.
__host__ __device__ __forceinline__ uint32_t mlx_to_frag_word(uint32_t w) {
  uint32_t o = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    o |= ((w >> (4 * b)) & 0xFu) << (8 * b);
    o |= ((w >> (4 * b + 16)) & 0xFu) << (8 * b + 4);
  }
  return o;
}

__host__ __device__ __forceinline__ uint32_t frag_to_mlx_word(uint32_t o) {
  uint32_t w = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    w |= ((o >> (8 * b)) & 0xFu) << (4 * b);
    w |= ((o >> (8 * b + 4)) & 0xFu) << (4 * b + 16);
  }
  return w;
}

// Packed fragment block of (tile t, group pair p): 288 u32 at word (t*GP + p)*288.
//   words [0, 256):   lane l, word 2j + h at 4l + 2j + h — row 16t + l%16, columns
//                     64(2p+j) + 32h + 8(l/16) + 0..7 (nibble order of mlx_to_frag_word);
//   words [256, 288): row r at 256 + 2r: scales of groups 2p, 2p+1 (low, high half),
//                     then biases of the same two groups.
constexpr int kBlockWords = 288;
constexpr int kBlockBytes = kBlockWords * 4;
constexpr int kSbOffsetBytes = 1024;

// kWords = kBlockWords: the full packed block (nibbles, then scales and biases); kWords = 256:
// the nibbles alone, [N, K/8] words like MLX's packs (the relayout of skinny_w4g64_relayout).
template <bool kForward, int kWords = kBlockWords>
__global__ void pack_kernel(uint32_t* __restrict__ w_mlx, uint16_t* __restrict__ sc, uint16_t* __restrict__ bi,
                            uint32_t* __restrict__ frag, int N, int K) {
  const int G = K >> 6, GP = K >> 7, KW = K >> 3;
  const size_t total = (size_t)(N >> 4) * GP * kWords;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int wi = (int)(i % kWords);
    const size_t blk = i / kWords;
    const int gp = (int)(blk % GP);
    const int t = (int)(blk / GP);
    if (wi < 256) {
      const int l = wi >> 2, j = (wi >> 1) & 1, h = wi & 1;
      const int row = t * 16 + (l & 15);
      const size_t wm = (size_t)row * KW + (2 * gp + j) * 8 + h * 4 + (l >> 4);
      if (kForward) frag[i] = mlx_to_frag_word(w_mlx[wm]);
      else w_mlx[wm] = frag_to_mlx_word(frag[i]);
    } else {
      const int r = (wi - 256) >> 1;
      uint16_t* src = ((wi - 256) & 1) ? bi : sc;
      const size_t e = (size_t)(t * 16 + r) * G + 2 * gp;
      if (kForward) frag[i] = (uint32_t)src[e] | ((uint32_t)src[e + 1] << 16);
      else {
        src[e] = (uint16_t)(frag[i] & 0xffffu);
        src[e + 1] = (uint16_t)(frag[i] >> 16);
      }
    }
  }
}

// Full packed blocks from a nibbles-only relayout and MLX-layout scales and biases: words
// [0, 256) of block (t, p) are the relayout's block, words [256, 288) as skinny_w4g64_pack.
__global__ void attach_kernel(const uint32_t* __restrict__ nib, const uint16_t* __restrict__ sc,
                              const uint16_t* __restrict__ bi, uint32_t* __restrict__ frag, int N, int K) {
  const int G = K >> 6, GP = K >> 7;
  const size_t total = (size_t)(N >> 4) * GP * kBlockWords;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int wi = (int)(i % kBlockWords);
    const size_t blk = i / kBlockWords;
    if (wi < 256) {
      frag[i] = nib[blk * 256 + wi];
    } else {
      const int gp = (int)(blk % GP), t = (int)(blk / GP);
      const int r = (wi - 256) >> 1;
      const uint16_t* src = ((wi - 256) & 1) ? bi : sc;
      const size_t e = (size_t)(t * 16 + r) * G + 2 * gp;
      frag[i] = (uint32_t)src[e] | ((uint32_t)src[e + 1] << 16);
    }
  }
}

// Eight codes of one fragment word -> the B operand: bf16 pairs (128 + e_2v, 128 + e_2v+1),
// built by v_perm_b32 from one code per byte and a 0x43 byte (bf16 128.0 = 0x4300, and
// 0x4300 | q = 128 + q exactly for q < 128).
__device__ __forceinline__ bf16x8_t unpack_nibbles(uint32_t w) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // e0 e1 e2 e3
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // e4 e5 e6 e7
  u32x4_t p;
  p.x = __builtin_amdgcn_perm(0x43434343u, lo, 0x04010400u);
  p.y = __builtin_amdgcn_perm(0x43434343u, lo, 0x04030402u);
  p.z = __builtin_amdgcn_perm(0x43434343u, hi, 0x04010400u);
  p.w = __builtin_amdgcn_perm(0x43434343u, hi, 0x04030402u);
  return __builtin_bit_cast(bf16x8_t, p);
}

// X fragments of one group pair: [group j][k half h].
struct XStage {
  bf16x8_t a[2][2];
};

// Weight side of one group pair for RF row tiles.
template <int RF>
struct WStage {
  u32x4_t w[RF];   // fragment words: (g0 h0, g0 h1, g1 h0, g1 h1)
  u32x2_t sb[RF];  // (scales of g0|g1, biases of g0|g1) for the lane's row
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // gfx9 raw buffer: stride 0, byte-granular range check, word 3 = 0x00020000
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// X for group pair gp: the lane's voffset selects (token, quad); rows >= M carry an
// out-of-range voffset and load zeros.
__device__ __forceinline__ void load_x(XStage& xs, __amdgpu_buffer_rsrc_t rx, uint32_t xoff, int gp) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      xs.a[j][h] = __builtin_bit_cast(
          bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(rx, xoff, (2 * gp + j) * 128 + h * 64, 0));
}

// Gated-norm-in (GN) operands of one group pair, which is one head of 128 values (K = heads x 128):
// the lane's fp32 y and bf16 z at the positions of its X fragment, [group j][k half h].
struct GStage {
  f32x4_t y[2][2][2];
  u32x4_t z[2][2];
};

__device__ __forceinline__ void load_g(GStage& g, __amdgpu_buffer_rsrc_t ry, uint32_t yoff, __amdgpu_buffer_rsrc_t rz,
                                       uint32_t zoff, int gp) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = (2 * gp + j) * 64 + h * 32;
      g.y[j][h][0] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ry, yoff, k * 4, 0));
      g.y[j][h][1] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ry, yoff, k * 4 + 16, 0));
      g.z[j][h] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rz, zoff, k * 2, 0));
    }
}

// X = bf16(rmsnorm(y) * w * silu(z)) over the head, bitwise what skinny_gated_rmsnorm writes. That
// kernel's lane i (one wave per token and head) squares values i and i + 64 in an fmaf chain, and
// wave_sum adds the 64 chains: pairs, quads and eight-lane groups inside each 16-lane row, the row
// sums, then (r0 + r1) + (r2 + r3). A lane here holds the values i = 8 quad + 32 h + e (e < 8) and
// i + 64 for both h: the two eight-value groups of that sum, which it adds in the same tree; the
// xor-16 exchange pairs the groups of one row and the xor-32 exchange the rows, each addition
// with the same two operands as there, so every lane of the token ends with the same sum.
__device__ __forceinline__ void gated_x(XStage& xs, const GStage& g, const u32x4_t (&w)[2][2], float eps) {
  float grp[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y0 = g.y[0][h][e >> 2][e & 3], y1 = g.y[1][h][e >> 2][e & 3];
      p[e] = fmaf(y1, y1, y0 * y0);
    }
    grp[h] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
  }
  const float r0 = grp[0] + __shfl_xor(grp[0], 16, 64), r1 = grp[1] + __shfl_xor(grp[1], 16, 64);
  const float ss = (r0 + __shfl_xor(r0, 32, 64)) + (r1 + __shfl_xor(r1, 32, 64));
  const float inv = rsqrtf(ss / 128.0f + eps);
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int e = 2 * q + b;
          const uint32_t zb = (g.z[j][h][q] >> (16 * b)) & 0xffffu, wb = (w[j][h][q] >> (16 * b)) & 0xffffu;
          const float zf = bf16_bits_to_f32(zb);
          const float gate = silu_gate(zf);
          word |= (uint32_t)f32_to_bf16_bits(g.y[j][h][e >> 2][e & 3] * inv * bf16_bits_to_f32(wb) * gate) << (16 * b);
        }
        o[q] = word;
      }
      xs.a[j][h] = __builtin_bit_cast(bf16x8_t, o);
    }
}

template <int RF>
__device__ __forceinline__ void load_w(WStage<RF>& ws, __amdgpu_buffer_rsrc_t rw, uint32_t woff, uint32_t sboff,
                                       int gp, int GP) {
#pragma unroll
  for (int r = 0; r < RF; ++r) {
    const int blk = (r * GP + gp) * kBlockBytes;
    ws.w[r] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, woff, blk, 0));
    ws.sb[r] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rw, sboff, blk, 0));
  }
}

template <int RF>
__device__ __forceinline__ void compute(const XStage& xs, const WStage<RF>& ws, f32x4_t (&acc)[RF],
                                        const bf16x8_t ones) {
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    f32x4_t xsum = mfma16x16x32(xs.a[j][0], ones, zero);
    xsum = mfma16x16x32(xs.a[j][1], ones, xsum);
#pragma unroll
    for (int r = 0; r < RF; ++r) {
      const uint32_t w0 = j ? ws.w[r].z : ws.w[r].x;
      const uint32_t w1 = j ? ws.w[r].w : ws.w[r].y;
      f32x4_t g = mfma16x16x32(xs.a[j][0], unpack_nibbles(w0), zero);
      g = mfma16x16x32(xs.a[j][1], unpack_nibbles(w1), g);
      const float s = __uint_as_float(j ? (ws.sb[r].x & 0xffff0000u) : (ws.sb[r].x << 16));
      const float b = __uint_as_float(j ? (ws.sb[r].y & 0xffff0000u) : (ws.sb[r].y << 16));
      const float bp = fmaf(-128.0f, s, b);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[r][i] = fmaf(s, g[i], acc[r][i]);
        acc[r][i] = fmaf(bp, xsum[i], acc[r][i]);
      }
    }
  }
}

__device__ __forceinline__ bf16x8_t ones_operand() {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
}

// LDS writes of this wave complete, then every wave of the workgroup meets. Global loads
// still in flight are not waited for (unlike __syncthreads()).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---------------------------------------------------------------------------------------------
// RF row tiles per wave; SK waves per workgroup split the K/128 group pairs as
// evenly as possible (wave w owns [w*GP/SK, (w+1)*GP/SK)). Each wave streams its pairs through
// a ring of NS stages; a stage holds one pair's weights, scales, biases AND X fragments, issued
// together NS pairs ahead of use. The pair consumed next is therefore always the oldest
// outstanding load, which is what the in-order vmcnt counter can wait for without stalling on
// younger prefetches. Refill rounds have no control flow around loads; loads past the wave's
// last pair repeat that pair (cache hits) and are not consumed.
//
// Epilogues (EPI): kPlain stores row tile t at columns 16t.. . The gate|up layouts pair tile
// 2j (gate rows 16j..) with tile 2j+1 (up rows 16j..) in one RF = 2 wave: kGluSplit stores
// them back at gate column 16j and up column N/2 + 16j (the unfused [gate | up] order);
// kSwiGlu stores silu(gate) * up, both rounded to bf16 first, at column 16j of an [M, N/2]
// output — bitwise what the activation kernel makes of the kGluSplit result.
//
// kPartial writes fp32 sums instead, one slice per K split: workgroup (g, s) of a grid with
// gridDim.y = S splits covers group pairs [s*GP/S, (s+1)*GP/S) and stores its tiles' sums at
// y32[(s*M + t)*ldy + column], unrounded; the consumer adds the S slices in split order. With
// S = 1 every pair assignment is the unsplit kernel's.
//
// kConv is kPlain for the fused Gated-DeltaNet input projection, with the mixer's short causal
// conv and SiLU applied to its first C columns (the conv channels q | k | v): a workgroup holds
// every token of its columns, so each channel's conv runs in the one workgroup that owns it. Per
// channel the sequence [conv state (KW-1 rows); bf16(y) of the M tokens] is staged in LDS, each
// token's output is bf16(silu(sum_j w_j seq[t+j])) with the taps accumulated oldest first (a draft
// tree's taps follow its parent pointers, as in skinny_gdn_conv_silu), the input rows go to the
// rollback window when one is given, and a chain moves the last KW-1 rows into the conv state:
// bitwise what skinny_gdn_conv_silu makes of the kPlain output. Columns from C on are stored as
// kPlain stores them.
//
// kSplitK is kPlain with S workgroups per row tile group, each over its share of the group pairs
// as in kPartial. Splits 0 .. S-2 publish their fp32 sums with device-coherent stores into a
// workspace whose words hold kEmpty until written; the last split (dispatched after every other,
// and waiting only on them, so it cannot deadlock) reads each word once it is no longer kEmpty,
// adds the slices in split order to its own sums, stores bf16 and puts kEmpty back. The data is its
// own readiness flag: no atomics, no fences, no wait for store completion.
//
// kSwiGluPublish is kSwiGlu for the gate|up half of the fused MLP launch (mlp_fused_kernel): the
// [M, N/2] output goes out with device-coherent (write-through) stores, the wave waits for them,
// then counts its 16 columns in ea.sync[column / 128], the group of 128 columns (one K pair of the
// down projection) that the launch's down waves wait for.
enum Epilogue { kPlain = 0, kGluSplit = 1, kSwiGlu = 2, kPartial = 3, kConv = 8, kSplitK = 9, kPublish = 10,
                kSwiGluPublish = 11 };
constexpr uint32_t kEmpty = 0xffffffffu;  // a split-K workspace word not yet written (a NaN no sum takes)
constexpr int kSpinLimit = 1 << 20;       // polls of a slice word before the last split gives up
constexpr int kMaxSplitK = 4;
// Words between the fused MLP launch's counters: 4160 bytes, so the counters polled by hundreds of
// waves fall on different memory channels (packed into a few cache lines, the polls saturated their
// channel and stalled every weight stream that crossed it).
constexpr int kSyncStride = 1040;
constexpr int kSyncSleep = 8;  // s_sleep between polls of a counter (64 clocks each)
constexpr int kSplitKHeaderWords = 4;     // the split-K workspace's header: the sticky error word + padding
constexpr int kConvKW = 4;       // conv taps (the kConv epilogue's kernel width)
constexpr int kConvTokens = 16;  // tokens per launch of the kConv epilogue

struct EpiArgs {
  // kSplitK: split slices
  float* part;
  // norm-in kernels: the rows the input is the RMSNorm of (see NormInLayout)
  const uint16_t* ni_h;     // [M][K] residual stream before the add
  const float* ni_parts;    // [ni_splits][M][K] fp32 slices of the residual projection (ni_splits 0: none)
  int ni_splits;
  const uint16_t* ni_w;     // [K] norm weight
  float ni_eps;
  uint16_t* ni_hout;        // [M][K] residual stream after the add, or NULL
  // gated-norm-in kernels (GN): X = the Gated-DeltaNet output norm of y and z (see gated_x)
  const float* gn_y;        // [M][K] fp32, row stride gn_ldy
  int gn_ldy;
  const uint16_t* gn_z;     // [M][K] bf16 gate, row stride gn_ldz
  int gn_ldz;
  const uint16_t* gn_w;     // [128] norm weight (the same for every head)
  float gn_eps;
  // the fused MLP launch: per-128-column arrival counters, then the consumer count (see mlp_fused_kernel)
  uint32_t* sync;
  int sync_groups;      // counters in sync (then the consumer count at sync[sync_groups])
  int sync_expect;      // arrivals per counter (16-column producers per 128 columns: 8)
  int sync_consumers;   // consumer workgroups of the launch
  // kConv
  int conv_C;
  uint16_t* conv_state;     // [KW-1][C]
  const uint16_t* conv_w;   // [C][KW]
  uint16_t* window;         // [KW-1+M][C] or NULL
  const int32_t* parent;    // draft tree: [M] parent node (-1 = the root's predecessor) or NULL
};

// Norm-in kernels (NI) take, instead of X, the rows X is the RMSNorm of: X = rmsnorm(v) * w with
// v = bf16(h + bf16(sum of the residual slices in split order)) (v = h without slices), every
// element and the sum of squares formed as skinny_rmsnorm_partials_bf16 forms them (a fused
// multiply-add chain per 8-value chunk, wave_sum per 64 chunks, the groups in order), so X is
// bitwise that kernel's output. Each workgroup stages h, the slices
// and w in LDS by LDS-DMA, issued before its weight ring so the two latencies overlap, and forms
// all of X there (every workgroup repeats this small amount of work: it replaces a launch);
// workgroup (0, 0) also stores v, the new residual stream. LDS images, 1 KB aligned:
struct NormInLayout {
  uint32_t h, p, w, t, inv, bytes;  // byte offsets of h [M][K], slices [S][M][K], w [K], chunk sums [M][K/8], 1/rms [16]
  __host__ __device__ static uint32_t up(uint32_t b) { return (b + 1023u) & ~1023u; }
  __host__ __device__ NormInLayout(int M, int K, int S) {
    h = 0;
    p = h + up((uint32_t)M * K * 2);
    w = p + up((uint32_t)S * M * K * 4);
    t = w + up((uint32_t)K * 2);
    inv = t + (((uint32_t)M * (K / 8) * 4 + 15u) & ~15u);
    bytes = inv + 64;
  }
};
constexpr int kNormInMaxM = 4;
constexpr int kMaxNormInTiles = 256;       // K <= 4096: one 8-value chunk per thread of the norm kernel
constexpr int kNormInWaves = 8;            // the norm kernel's waves (512 threads)
constexpr uint32_t kNormInMaxLds = 96 * 1024;

// X fragments of group pair gp from the LDS rows (tokens >= M: zeros).
__device__ __forceinline__ void load_x_lds(XStage& xs, const uint16_t* xl, int tok, int quad, int M, int K, int gp) {
  const bf16x8_t zero = __builtin_bit_cast(bf16x8_t, u32x4_t{0u, 0u, 0u, 0u});
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      xs.a[j][h] = tok < M ? *reinterpret_cast<const bf16x8_t*>(xl + (size_t)tok * K + (2 * gp + j) * 64 + h * 32 + quad * 8)
                           : zero;
}

// The wave-X matmul of workgroup (bx, by) = (row tile group, K split): the body of qmm_wavex_kernel,
// shared with the q|k|v projection + attention kernel below.
//
// The K split's pairs are cut into SK * VS groups of consecutive pairs (the same cut for every VS);
// wave w accumulates groups w VS .. w VS + VS - 1, each from zero in its own accumulators, and the
// group sums are added in group order, so the result depends on SK * VS only. VS > 1 (one wave,
// groups of exactly GS pairs, the loop unrolled so that every pair's accumulator is static)
// therefore gives bitwise the products of the SK * VS-wave tile with fewer waves in flight: the
// launcher picks the physical form per token count.
//
// IW > 1 (one-wave tiles only, SK = 1): the workgroup holds IW independent instances, one per wave,
// each with its own bx (the caller's) and its own slot of the reduction LDS; no workgroup barrier.
// WX: X is produced by other workgroups of the same launch (mlp_fused_kernel). The weight ring's
// first loads are issued at once; the wave then polls ea.sync's counters of exactly its own K pairs
// (device-coherent loads, bounded: a wait that gives up makes the wave's sums NaN, never a hang),
// and only then loads X. After the reduction the workgroup adds itself to the consumer count, and
// the last consumer puts every counter back to 0, so each launch starts from zeros.
template <int RF, int SK, int NS, int EPI, bool NI = false, bool GN = false, int VS = 1, int GS = 0, int IW = 1,
          bool WX = false>
__device__ __forceinline__ void wavex_body(int bx, int by, const uint16_t* __restrict__ x, int M, int K, int ldx,
                                           const uint32_t* __restrict__ wfrag, int N, int S, uint16_t* __restrict__ y,
                                           int ldy, const EpiArgs ea) {
  constexpr int B = EPI;
  static_assert(B == kPlain || B == kPartial || B == kConv || B == kSplitK || B == kPublish || RF == 2,
                "gate|up epilogues pair two row tiles per wave");
  static_assert(VS == 1 || (SK == 1 && !NI && !GN && GS >= 1),
                "several K groups per wave only in one-wave plain-input tiles of a fixed group size");
  static_assert(IW == 1 || (SK == 1 && !NI && !GN && B == kSwiGluPublish), "independent waves: one-wave SwiGLU tiles");
  static_assert(!WX || (!NI && !GN && VS == 1 && B == kPartial), "waiting for X: plain-input split-K slices");
  static_assert(B != kSwiGluPublish || IW > 1, "the publishing SwiGLU epilogue runs in the fused MLP launch");
  const int GP = K >> 7;
  const int lane = threadIdx.x & 63;
  const int pwave = wave_id();                   // the physical wave in the workgroup
  const int wave = IW > 1 ? 0 : pwave;           // the wave's place among the tile's SK waves
  const int tile0 = bx * RF;
  const int tok = lane & 15;
  const int quad = lane >> 4;
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(reinterpret_cast<const char*>(wfrag) + (size_t)tile0 * GP * kBlockBytes, (uint32_t)(RF * GP * kBlockBytes));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((size_t)M * ldx * 2));
  const uint32_t xoff = tok < M ? (uint32_t)(tok * ldx + quad * 8) * 2u : 0x40000000u;
  const uint32_t woff = (uint32_t)lane * 16u;
  const uint32_t sboff = kSbOffsetBytes + (uint32_t)tok * 8u;
  const bf16x8_t ones = ones_operand();

  // S = gridDim.y K splits, passed as an argument: it is among the preloaded argument dwords,
  // where reading the grid size would wait on a fetch before the first load.
  const int pb = by * GP / S;  // this workgroup's K split
  const int GPs = (by + 1) * GP / S - pb;
  constexpr int G = SK * VS;  // K groups of the split
  const int gpa = pb + wave * VS * GPs / G;
  const int npairs = pb + (wave + 1) * VS * GPs / G - gpa;  // >= VS: the host keeps SK * VS <= pairs per split
  // (VS > 1: the host launches it only where npairs = VS * GS)
  const int last = gpa + npairs - 1;

  // NI: the rows first. With a thread per 16-column task (M * K/16 <= 64 SK) each thread with a
  // task loads its h, the slices that exist and w into registers (whether a load is issued depends
  // on the thread index and the split count only, never on loaded data, so nothing waits on it);
  // otherwise h, the slices and w go to LDS by LDS-DMA (1 KB per instruction, zeros past a buffer's
  // end). Either way these loads are older than the weight ring's.
  extern __shared__ __attribute__((aligned(16))) char ni_lds[];
  const NormInLayout nil(NI ? M : 0, NI ? K : 0, NI ? ea.ni_splits : 0);
  const bool ni_regs = NI && M * (K >> 4) <= 64 * SK;
  u32x4_t ni_rh[2], ni_rw[2];
  f32x4_t ni_rp[kMaxSplitK][4];
  if constexpr (NI) {
    if (ni_regs) {
      if ((int)threadIdx.x < M * (K >> 4)) {
        const int base = (int)threadIdx.x * 16, col = base % K;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          ni_rh[q] = *reinterpret_cast<const u32x4_t*>(ea.ni_h + base + 8 * q);
          ni_rw[q] = *reinterpret_cast<const u32x4_t*>(ea.ni_w + col + 8 * q);
        }
#pragma unroll
        for (int sp = 0; sp < kMaxSplitK; ++sp) {
          if (sp < ea.ni_splits) {
            const float* src = ea.ni_parts + (size_t)sp * M * K + base;
#pragma unroll
            for (int q = 0; q < 4; ++q) ni_rp[sp][q] = *reinterpret_cast<const f32x4_t*>(src + 4 * q);
          }
        }
      }
    } else {
      auto dma = [&](const void* src, uint32_t bytes, uint32_t lds_off) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, bytes);
        for (uint32_t i = (uint32_t)wave; i * 1024u < bytes; i += SK)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(ni_lds + lds_off + i * 1024u),
                                                   16, (uint32_t)lane * 16u, i * 1024u, 0, 0);
      };
      dma(ea.ni_h, (uint32_t)M * K * 2, nil.h);
      if (ea.ni_splits > 0) dma(ea.ni_parts, (uint32_t)ea.ni_splits * M * K * 4, nil.p);
      dma(ea.ni_w, (uint32_t)K * 2, nil.w);
    }
    asm volatile("" ::: "memory");  // the weight loads below stay younger than these
    __builtin_amdgcn_sched_barrier(0);
  }

  WStage<RF> ws[NS];
  XStage xs[NS];
  // GN: y and z in place of X (tokens >= M read past the buffers' ranges, as zeros), the norm
  // weight at this lane's fragment positions once.
  GStage gs[GN ? NS : 1];
  u32x4_t gw[2][2];
  __amdgpu_buffer_rsrc_t ry = rx, rz = rx;
  uint32_t yoff = 0, zoff = 0;
  if constexpr (GN) {
    ry = make_rsrc(ea.gn_y, (uint32_t)((size_t)M * ea.gn_ldy * 4));
    rz = make_rsrc(ea.gn_z, (uint32_t)((size_t)M * ea.gn_ldz * 2));
    yoff = tok < M ? (uint32_t)(tok * ea.gn_ldy + quad * 8) * 4u : 0x40000000u;
    zoff = tok < M ? (uint32_t)(tok * ea.gn_ldz + quad * 8) * 2u : 0x40000000u;
  }
#pragma unroll
  for (int p = 0; p < NS; ++p) {
    const int gp = min(gpa + p, last);
    load_w<RF>(ws[p], rw, woff, sboff, gp, GP);
    if constexpr (GN)
      load_g(gs[p], ry, yoff, rz, zoff, gp);
    else if constexpr (!NI && !WX)
      load_x(xs[p], rx, xoff, gp);
  }
  bool wx_ok = true;
  if constexpr (WX) {
    // The weight ring is in flight; wait for this wave's K pairs (lane i: pair gpa + i, the host
    // keeps npairs <= 64), then load their X.
    const bool mine = lane < npairs;
    int polls = 0;
    while (true) {
      const uint32_t c = mine ? __hip_atomic_load(ea.sync + (size_t)(gpa + lane) * kSyncStride, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT)
                              : (uint32_t)ea.sync_expect;
      if (__builtin_amdgcn_ballot_w64(c != (uint32_t)ea.sync_expect) == 0) break;
      if (++polls > kSpinLimit) {
        wx_ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(kSyncSleep);
    }
    asm volatile("" ::: "memory");  // no X load moves above the wait
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < NS; ++p) load_x(xs[p], rx, xoff, min(gpa + p, last));
  }
  if constexpr (GN) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) gw[j][h] = *reinterpret_cast<const u32x4_t*>(ea.gn_w + j * 64 + h * 32 + quad * 8);
  }

  if constexpr (NI) {
    // The LDS-DMA loads are the oldest; waiting until only the ring's 2 * RF * NS loads remain
    // waits for them alone. Then: v and the chunk sums (pass 1), 1/rms per token (pass 2, wave 0),
    // X = bf16(v * inv * w) in place of v (pass 3).
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * RF * NS) : "memory");
    lds_barrier();
    uint16_t* hl = reinterpret_cast<uint16_t*>(ni_lds + nil.h);
    const float* pl = reinterpret_cast<const float*>(ni_lds + nil.p);
    const uint16_t* wl = reinterpret_cast<const uint16_t*>(ni_lds + nil.w);
    float* tl = reinterpret_cast<float*>(ni_lds + nil.t);
    float* il = reinterpret_cast<float*>(ni_lds + nil.inv);
    const int T = K >> 4, NSP = ea.ni_splits;
    const bool store_h = ea.ni_hout != nullptr && bx == 0 && by == 0;
    // Pass 1 per 16-column task: v (into LDS over h on the LDS path, kept in registers on the
    // register path), h_out, and the sums of squares of its two 8-value chunks.
    float vr[16];
    auto form_v = [&](int task, float (&v)[16], const u32x4_t (&hw)[2], auto&& slice) {
      const int base = task * 16;
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          v[8 * q + e] = bf16_bits_to_f32((e & 1) ? (hw[q][e >> 1] >> 16) : (hw[q][e >> 1] & 0xffffu));
      if (NSP > 0) {
        float r[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) r[e] = slice(0, e);
#pragma unroll
        for (int sp = 1; sp < kMaxSplitK; ++sp)
          if (sp < NSP)
#pragma unroll
            for (int e = 0; e < 16; ++e) r[e] += slice(sp, e);
#pragma unroll
        for (int e = 0; e < 16; ++e)
          v[e] = bf16_bits_to_f32(f32_to_bf16_bits(v[e] + bf16_bits_to_f32(f32_to_bf16_bits(r[e]))));
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        u32x4_t o;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[i] = (uint32_t)f32_to_bf16_bits(v[8 * q + 2 * i]) | ((uint32_t)f32_to_bf16_bits(v[8 * q + 2 * i + 1]) << 16);
        if (!ni_regs) *reinterpret_cast<u32x4_t*>(hl + base + 8 * q) = o;
        if (store_h) *reinterpret_cast<u32x4_t*>(ea.ni_hout + base + 8 * q) = o;
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {  // the norm kernel's per-thread chains, one per 8-value chunk
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[8 * q + e], v[8 * q + e], ss);
        tl[2 * task + q] = ss;
      }
    };
    if (ni_regs) {
      if ((int)threadIdx.x < M * T)
        form_v((int)threadIdx.x, vr, ni_rh, [&](int sp, int e) { return ni_rp[sp][e >> 2][e & 3]; });
    } else {
      for (int task = (int)threadIdx.x; task < M * T; task += 64 * SK) {
        const int base = task * 16;
        u32x4_t hw[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) hw[q] = *reinterpret_cast<const u32x4_t*>(hl + base + 8 * q);
        float v[16];
        form_v(task, v, hw, [&](int sp, int e) { return pl[(size_t)sp * M * K + base + e]; });
      }
    }
    lds_barrier();
    if (wave == 0) {
      // Per token: wave_sum over each 64-chunk group (a wave of the norm kernel), the groups added
      // in order from 0 (groups past the row add 0).
      const int nchunk = K >> 3;
      for (int t = 0; t < M; ++t) {
        float c[kNormInWaves];
#pragma unroll
        for (int w = 0; w < kNormInWaves; ++w) {
          const int ch = 64 * w + lane;
          c[w] = tl[t * nchunk + min(ch, nchunk - 1)];
          c[w] = ch < nchunk ? c[w] : 0.f;
        }
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < kNormInWaves; ++w) acc += wave_sum(c[w]);
        if (lane == 0) il[t] = rsqrtf(acc / (float)K + ea.ni_eps);
      }
    }
    lds_barrier();
    // Pass 3: X = bf16(v * inv * w) into the LDS rows.
    auto form_x = [&](int task, const float (&v)[16], const u32x4_t (&ww)[2]) {
      const int t = task / T, base = task * 16;
      const float inv = il[t];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        u32x4_t o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float w0 = bf16_bits_to_f32(ww[q][i] & 0xffffu), w1 = bf16_bits_to_f32(ww[q][i] >> 16);
          o[i] = (uint32_t)f32_to_bf16_bits(v[8 * q + 2 * i] * inv * w0) |
                 ((uint32_t)f32_to_bf16_bits(v[8 * q + 2 * i + 1] * inv * w1) << 16);
        }
        *reinterpret_cast<u32x4_t*>(hl + base + 8 * q) = o;
      }
    };
    if (ni_regs) {
      if ((int)threadIdx.x < M * T) form_x((int)threadIdx.x, vr, ni_rw);
    } else {
      for (int task = (int)threadIdx.x; task < M * T; task += 64 * SK) {
        const int base = task * 16, col = base % K;
        float v[16];
        u32x4_t ww[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const u32x4_t vw = *reinterpret_cast<const u32x4_t*>(hl + base + 8 * q);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[8 * q + e] = bf16_bits_to_f32((e & 1) ? (vw[e >> 1] >> 16) : (vw[e >> 1] & 0xffffu));
          ww[q] = *reinterpret_cast<const u32x4_t*>(wl + col + 8 * q);
        }
        form_x(task, v, ww);
      }
    }
    lds_barrier();
#pragma unroll
    for (int p = 0; p < NS; ++p) load_x_lds(xs[p], hl, tok, quad, M, K, min(gpa + p, last));
  }

  // kConv: this workgroup's conv taps (16·RF channels × KW bf16, channel-major) and its columns of
  // the KW-1 conv-state rows into LDS, by LDS-DMA (4 bytes per lane, 256 B per instruction;
  // channels from C on are past the buffers' ranges and read as zeros). Issued after the ring's
  // first loads: its arguments lie past the preloaded ones, and only the epilogue needs it.
  constexpr int kCwInstr = B == kConv ? (16 * RF * kConvKW * 2 + 255) / 256 : 1;
  __shared__ __attribute__((aligned(16))) uint16_t cw_lds[kCwInstr * 128];
  __shared__ __attribute__((aligned(16))) uint16_t cs_lds[B == kConv ? kConvKW - 1 : 1][128];
  if constexpr (B == kConv) {
    const int c0 = tile0 * 16;
    if (c0 < ea.conv_C) {
      const uint32_t live = (uint32_t)min(16 * RF, ea.conv_C - c0);
      for (int i = wave; i < kCwInstr + kConvKW - 1; i += SK) {
        if (i < kCwInstr) {
          const __amdgpu_buffer_rsrc_t rc = make_rsrc(ea.conv_w + (size_t)c0 * kConvKW, live * kConvKW * 2u);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (__attribute__((address_space(3))) void*)&cw_lds[i * 128], 4,
                                                   (uint32_t)lane * 4u, (uint32_t)i * 256u, 0, 0);
        } else {
          const int j = i - kCwInstr;
          const __amdgpu_buffer_rsrc_t rc = make_rsrc(ea.conv_state + (size_t)j * ea.conv_C + c0, live * 2u);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (__attribute__((address_space(3))) void*)&cs_lds[j][0], 4,
                                                   (uint32_t)lane * 4u, 0, 0, 0);
        }
      }
    }
  }

  f32x4_t acc[RF];
#pragma unroll
  for (int r = 0; r < RF; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  f32x4_t accv[VS > 1 ? VS : 1][RF];
  if constexpr (VS > 1) {
    // Every pair at a static ring stage and group accumulator; groups summed in order from zero,
    // as the workgroup sum of a VS-wave tile adds its waves.
#pragma unroll
    for (int v = 0; v < VS; ++v)
#pragma unroll
      for (int r = 0; r < RF; ++r) accv[v][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < VS * GS; ++i) {
      const int p = i % NS;
      compute<RF>(xs[p], ws[p], accv[i / GS], ones);
      if (i + NS < VS * GS) {
        const int gp = min(gpa + i + NS, last);
        load_w<RF>(ws[p], rw, woff, sboff, gp, GP);
        load_x(xs[p], rx, xoff, gp);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < RF; ++r) {
      f32x4_t t = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < VS; ++v) t += accv[v][r];
      acc[r] = t;
    }
  }
  int base = VS > 1 ? npairs : 0;
  for (; base + NS < npairs; base += NS) {  // rounds that refill the ring
#pragma unroll
    for (int p = 0; p < NS; ++p) {
      if constexpr (GN) gated_x(xs[p], gs[p], gw, ea.gn_eps);
      compute<RF>(xs[p], ws[p], acc, ones);
      const int gp = min(gpa + base + p + NS, last);
      load_w<RF>(ws[p], rw, woff, sboff, gp, GP);
      if constexpr (GN)
        load_g(gs[p], ry, yoff, rz, zoff, gp);
      else if constexpr (NI)
        load_x_lds(xs[p], reinterpret_cast<const uint16_t*>(ni_lds + nil.h), tok, quad, M, K, gp);
      else
        load_x(xs[p], rx, xoff, gp);
      // Keep the ring order: without this the scheduler hoists the next pair's arithmetic above
      // these loads, and each round then waits with only its own pair in flight.
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int p = 0; p < NS; ++p)  // final round: 1..NS pairs left, all in the ring
    if (VS == 1 && base + p < npairs) {
      if constexpr (GN) gated_x(xs[p], gs[p], gw, ea.gn_eps);
      compute<RF>(xs[p], ws[p], acc, ones);
    }

  if constexpr (WX) {
    if (!wx_ok) {  // a pair that never arrived: NaN sums, not a hang
#pragma unroll
      for (int r = 0; r < RF; ++r) acc[r] = f32x4_t{NAN, NAN, NAN, NAN};
    }
  }
  // Split-K reduction across the SK waves, in wave order (IW > 1: each instance its own slot).
  __shared__ float red[SK * IW][RF][4][64];
  const int rslot = IW > 1 ? pwave : 0;
#pragma unroll
  for (int r = 0; r < RF; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[rslot + wave][r][j][lane] = acc[r][j];
  if constexpr (B == kConv) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's LDS-DMA has landed
  if constexpr (IW > 1)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave reads back only its own slot
  else
    __syncthreads();
  if constexpr (WX) {
    // Every X load of the workgroup is behind it: count it as a consumer; the last one resets.
    if (threadIdx.x == 0) {
      uint32_t* done = ea.sync + (size_t)ea.sync_groups * kSyncStride;
      const uint32_t prev = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (prev == (uint32_t)ea.sync_consumers - 1u) {
        for (int g = 0; g < ea.sync_groups; ++g)
          __hip_atomic_store(ea.sync + (size_t)g * kSyncStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  auto total = [&](int r, int t, int n) {  // wave-order sum of (tile r, token t, row n)
    const int l = (t >> 2) * 16 + n, j = t & 3;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < SK; ++w) v += red[rslot + w][r][j][l];
    return v;
  };
  if constexpr (B == kConv) {
    // Rows i of seq_lds: the KW-1 conv-state rows, then bf16(y) of the M tokens; one column per
    // channel of this workgroup. Phase 1 stages them (and the window, and the plain columns),
    // phase 2 runs the conv per (token, channel) and moves a chain's last KW-1 rows to the state.
    constexpr int CH = 16 * RF;
    __shared__ uint16_t seq_lds[kConvKW - 1 + kConvTokens][CH];
    __shared__ int par_lds[kConvTokens];
    const int C = ea.conv_C;
    const int rows = kConvKW - 1 + M;
    if (ea.parent && (int)threadIdx.x < M) par_lds[threadIdx.x] = ea.parent[threadIdx.x];
    for (int idx = threadIdx.x; idx < rows * CH; idx += 64 * SK) {
      const int ch = idx % CH, i = idx / CH;
      const int n = ch & 15, r = ch >> 4;
      const size_t col = (size_t)(tile0 + r) * 16 + n;
      const bool conv = col < (size_t)C;
      uint16_t v;
      if (i < kConvKW - 1) {
        if (!conv) continue;
        v = cs_lds[i][ch];
      } else {
        v = f32_to_bf16_bits(total(r, i - (kConvKW - 1), n));
        if (!conv) {
          y[(size_t)(i - (kConvKW - 1)) * ldy + col] = v;
          continue;
        }
      }
      seq_lds[i][ch] = v;
      if (ea.window) ea.window[(size_t)i * C + col] = v;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < M * CH; idx += 64 * SK) {
      const int ch = idx % CH, t = idx / CH;
      const size_t col = (size_t)(tile0 + (ch >> 4)) * 16 + (ch & 15);
      if (col >= (size_t)C) continue;
      int at[kConvKW];  // row of tap j: the input KW-1-j steps back along the chain or the ancestors
      if (ea.parent) {
        int a = t;
#pragma unroll
        for (int j = kConvKW - 1; j >= 0; --j) {
          at[j] = kConvKW - 1 + a;
          a = a >= 0 ? par_lds[a] : a - 1;
        }
      } else {
#pragma unroll
        for (int j = 0; j < kConvKW; ++j) at[j] = t + j;
      }
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < kConvKW; ++j)
        acc = fmaf(bf16_bits_to_f32(cw_lds[ch * kConvKW + j]), bf16_bits_to_f32(seq_lds[at[j]][ch]), acc);
      y[(size_t)t * ldy + col] = f32_to_bf16_bits(acc / (1.0f + expf(-acc)));
    }
    if (!ea.parent) {
      for (int idx = threadIdx.x; idx < (kConvKW - 1) * CH; idx += 64 * SK) {
        const int ch = idx % CH, j = idx / CH;
        const size_t col = (size_t)(tile0 + (ch >> 4)) * 16 + (ch & 15);
        if (col < (size_t)C) ea.conv_state[(size_t)j * C + col] = seq_lds[M + j][ch];
      }
    }
  } else if constexpr (B == kSplitK) {
    // workspace ea.part: a 16-byte header (word 0: the sticky error word, kEmpty while no last
    // split has given up), then S-1 slices [16 tokens][N] fp32
    constexpr int kElems = 16 * RF * 16;
    constexpr int kPer = (kElems + 64 * SK - 1) / (64 * SK);
    const int sp_own = by;
    const bool last = sp_own == S - 1;
    uint32_t* const err_word = reinterpret_cast<uint32_t*>(ea.part);
    // A workspace that a timed-out call left behind may still receive a late slice, so its words
    // prove nothing: every later call's output is NaN until the caller replaces the workspace.
    const bool poisoned =
        last && __hip_atomic_load(err_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != kEmpty;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int idx = (int)threadIdx.x + k * 64 * SK;
      const int n = idx & 15, r = (idx >> 4) % RF, t = idx / (16 * RF);
      const bool valid = idx < kElems && t < M;
      const size_t col = (size_t)(tile0 + r) * 16 + n;
      const float v = valid ? total(r, t, n) : 0.f;
      float* slot = ea.part + kSplitKHeaderWords + (size_t)t * N + col;  // slice sp at + sp * 16 * N
      if (!last) {
        if (valid)
          __hip_atomic_store(slot + (size_t)sp_own * 16 * N, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        continue;
      }
      float u[kMaxSplitK - 1];
#pragma unroll
      for (int sp = 0; sp < kMaxSplitK - 1; ++sp)
        u[sp] = (valid && sp < S - 1) ? __hip_atomic_load(slot + (size_t)sp * 16 * N, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                                      : 0.f;
      bool ok = true;
#pragma unroll
      for (int sp = 0; sp < kMaxSplitK - 1; ++sp) {
        if (sp >= S - 1) break;
        int polls = 0;
        while (__builtin_amdgcn_ballot_w64(valid && __float_as_uint(u[sp]) == kEmpty) != 0) {
          if (++polls > kSpinLimit) {  // a slice that never arrives ends with NaN, not a hang
            ok = false;
            break;
          }
          __builtin_amdgcn_s_sleep(2);
          if (valid && __float_as_uint(u[sp]) == kEmpty)
            u[sp] = __hip_atomic_load(slot + (size_t)sp * 16 * N, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (!valid) continue;
      float sum = u[0];
#pragma unroll
      for (int sp = 1; sp < kMaxSplitK - 1; ++sp)
        if (sp < S - 1) sum += u[sp];
      sum += v;
      y[(size_t)t * ldy + col] = ok && !poisoned ? f32_to_bf16_bits(sum) : (uint16_t)0x7fc0u;
      if (!ok) {
        // A slice that never arrived may still be stored later: leave every word as it is and
        // mark the workspace, rather than reset words a late store would then make look valid.
        __hip_atomic_store(err_word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        continue;
      }
#pragma unroll
      for (int sp = 0; sp < kMaxSplitK - 1; ++sp)
        if (sp < S - 1)
          __hip_atomic_store(slot + (size_t)sp * 16 * N, __uint_as_float(kEmpty), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    }
  } else if constexpr (B == kSwiGlu) {
    for (int idx = threadIdx.x; idx < 16 * 16; idx += 64 * SK) {
      const int n = idx & 15, t = idx >> 4;
      if (t >= M) break;
      const float g = bf16_bits_to_f32(f32_to_bf16_bits(total(0, t, n)));
      const float u = bf16_bits_to_f32(f32_to_bf16_bits(total(1, t, n)));
      y[(size_t)t * ldy + (size_t)bx * 16 + n] = silu_mul_bf16(g, u);
    }
  } else if constexpr (B == kSwiGluPublish) {
    // kSwiGlu's values, stored write-through; then this wave's 16 columns count as arrived.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int idx = lane + 64 * k;
      const int n = idx & 15, t = idx >> 4;
      if (t < M) {
        const float g = bf16_bits_to_f32(f32_to_bf16_bits(total(0, t, n)));
        const float u = bf16_bits_to_f32(f32_to_bf16_bits(total(1, t, n)));
        __hip_atomic_store(y + (size_t)t * ldy + (size_t)bx * 16 + n, silu_mul_bf16(g, u), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // every store of the wave has completed
    if (lane == 0)
      __hip_atomic_fetch_add(ea.sync + (size_t)(bx >> 3) * kSyncStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    // Output element (token t, tile r, row n) with n fastest so stores run along rows.
    for (int idx = threadIdx.x; idx < 16 * RF * 16; idx += 64 * SK) {
      const int n = idx & 15;
      const int r = (idx >> 4) % RF;
      const int t = idx / (16 * RF);
      if (t >= M) break;  // idx grows with t
      const size_t col = B == kGluSplit ? (size_t)r * (N >> 1) + (size_t)bx * 16 + n
                                        : (size_t)(tile0 + r) * 16 + n;
      if constexpr (B == kPartial)
        reinterpret_cast<float*>(y)[((size_t)by * M + t) * ldy + col] = total(r, t, n);
      else if constexpr (B == kPublish)  // device-coherent: read by other workgroups of the launch
        __hip_atomic_store(y + (size_t)t * ldy + col, f32_to_bf16_bits(total(r, t, n)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      else
        y[(size_t)t * ldy + col] = f32_to_bf16_bits(total(r, t, n));
    }
  }
}

// The MLP sublayer of the 36-layer decoders in one launch, from two tokens on: workgroups
// [0, n_prod) each run one one-wave instance of the gate|up + SwiGLU tile in their first wave (the
// one-wave form of the 4-group tile over K = 2560, bitwise the gate|up launch; the other waves leave
// at once, so the instances spread over every CU as the gate|up launch's one-wave workgroups do —
// four per workgroup put them on 152 of the 256 CUs and made the phase 1.7x longer), publishing
// [M, F] into `act`;
// the rest are the down projection's split-K tiles (3 splits, rf 2, 4 waves, ring 3; bitwise its
// partial launch), which issue their weight rings at once and wait only for the 128-column groups of
// `act` their waves read. The producers are dispatched first and wait on nothing, so no wait depends
// on a workgroup that has not started.
constexpr int kMlpProdTiles = 1;  // one-wave gate|up instances per producer workgroup

__global__ __launch_bounds__(256) void mlp_fused_kernel(const uint16_t* __restrict__ x, int M, int K, int ldx,
                                                        const uint32_t* __restrict__ wgu, int F,
                                                        const uint32_t* __restrict__ wdn, int N, int S,
                                                        int n_prod, uint16_t* __restrict__ act,
                                                        float* __restrict__ part, const EpiArgs ea) {
  if ((int)blockIdx.x < n_prod) {
    if (wave_id() >= kMlpProdTiles) return;
    wavex_body<2, 1, 4, kSwiGluPublish, false, false, 4, 5, 4>((int)blockIdx.x * kMlpProdTiles + wave_id(), 0, x, M,
                                                             K, ldx, wgu, 2 * F, 1, act, F, ea);
  } else {
    const int c = (int)blockIdx.x - n_prod, groups = (N / 16) / 2;
    wavex_body<2, 4, 3, kPartial, false, false, 1, 0, 1, true>(c % groups, c / groups, act, M, F, F, wdn, N, S,
                                                              reinterpret_cast<uint16_t*>(part), N, ea);
  }
}

template <int RF, int SK, int NS, int EPI, bool NI = false, bool GN = false, int VS = 1, int GS = 0>
__global__ __launch_bounds__(64 * SK) void qmm_wavex_kernel(const uint16_t* __restrict__ x, int M, int K, int ldx,
                                                            const uint32_t* __restrict__ wfrag, int N, int S,
                                                            uint16_t* __restrict__ y, int ldy, const EpiArgs ea) {
  wavex_body<RF, SK, NS, EPI, NI, GN, VS, GS>((int)blockIdx.x, (int)blockIdx.y, x, M, K, ldx, wfrag, N, S, y, ldy, ea);
}

// ---------------------------------------------------------------------------------------------
// The q|k|v projection and the attention's chunk stage in one launch. Workgroups [0, n_proj) are
// the projection (the wave-X matmul of the table's tile, storing its rows with device-coherent
// stores into the hand-off buffer `qkv`, whose 16-bit words hold 0xFFFF until written); the
// workgroups after them are the attention chunks (c, h), c fastest, as attn_chunk_kernel's grid.
// A chunk workgroup reads the device position and issues its chunk's loads at once, in the shadow
// of the projection's weight stream, and then waits for just the rows it needs (the wait form of
// attn_chunk_body). The host launches it only when every workgroup of the grid fits on the GPU at
// once, so no wait depends on a workgroup that has not started; each wait is bounded besides.
struct QkvAttnArgs {
  FusedArgs fa;  // fa.ldq: the hand-off buffer's row stride
  int Hq, Hkv, maxlen, nch;
  float scale;
  uint16_t* kc;
  uint16_t* vt;
  const int32_t* tree;
  float* part_o;
  float* part_ml;
};

template <int RF, int SK, int NS>
__global__ __launch_bounds__(64 * SK) void qkv_attn_kernel(const int32_t* __restrict__ pos0, const uint16_t* __restrict__ x,
                                                           const uint32_t* __restrict__ wfrag, uint16_t* __restrict__ qkv,
                                                           int M, int K, int ldx, int N, int n_proj, const QkvAttnArgs aa) {
  static_assert(SK == kWaves, "the projection's and the attention's workgroups have one size");
  if ((int)blockIdx.x < n_proj) {
    wavex_body<RF, SK, NS, kPublish>((int)blockIdx.x, 0, x, M, K, ldx, wfrag, N, 1, qkv, aa.fa.ldq, EpiArgs{});
    return;
  }
  const int a = (int)blockIdx.x - n_proj;
  attn_chunk_body<true, true>(a % aa.nch, a / aa.nch, pos0, qkv, aa.fa, M, aa.Hq, aa.Hkv, aa.kc, aa.vt, aa.maxlen,
                              aa.scale, aa.tree, aa.part_o, aa.part_ml, aa.nch);
}

using QkvAttnKernel = void (*)(const int32_t*, const uint16_t*, const uint32_t*, uint16_t*, int, int, int, int, int,
                               const QkvAttnArgs);

// Instances: the q|k|v tile of the 36-layer decoders (2560 x 6144: rf 2, 4 waves, ring of 3).
QkvAttnKernel pick_qkv_attn(const skinny_qmm_tile& t) {
  if (t.kind != SKINNY_QMM_WAVE_X || t.waves != kWaves) return nullptr;
  if (t.rf == 2 && t.ns == 3) return qkv_attn_kernel<2, 4, 3>;
  return nullptr;
}

// ---------------------------------------------------------------------------------------------
// Slab-X kernel. The `waves` waves of a workgroup own different row tiles (wave w: tiles
// (b*waves + w)*RF .. +RF) and each walks ALL K/128 group pairs, so no cross-wave reduction is
// needed. X for the whole K is staged once per workgroup in an LDS slab by LDS-DMA buffer loads
// (buffer_load_dwordx4 ... lds, no VGPRs): instruction i = 4p + 2j + h writes 64 16-byte chunks,
// lane l = 16*quad + token receiving x[token][128p + 64j + 32h + 8quad .. +8] — exactly the A
// fragment lane l reads back, so the reads are conflict-free; tokens >= M are out of the buffer
// range and land as zeros. X then crosses the vector memory path once per workgroup rather than
// once per wave. Suits wide N with K small enough for the slab (4 KB per group pair).
template <int RF, int NS, int EPI>
__global__ __launch_bounds__(512) void qmm_slab_kernel(const uint16_t* __restrict__ x, int M, int K, int ldx,
                                                       const uint32_t* __restrict__ wfrag, int N, int,
                                                       uint16_t* __restrict__ y, int ldy, const EpiArgs) {
  static_assert(EPI == kPlain || RF == 2, "gate|up epilogues pair two row tiles per wave");
  extern __shared__ u32x4_t slab[];
  const int W = blockDim.x >> 6;
  const int GP = K >> 7, T = N >> 4;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int tok = lane & 15, quad = lane >> 4;
  const int tile0 = (blockIdx.x * W + wave) * RF;
  const bool active = tile0 < T;  // the host keeps T % RF == 0

  // 1. The slab: GP*4 DMA instructions shared round-robin by the waves.
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((size_t)M * ldx * 2));
  const uint32_t xoff = tok < M ? (uint32_t)(tok * ldx + quad * 8) * 2u : 0x40000000u;
  for (int i = wave; i < GP * 4; i += W)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)&slab[i * 64], 16, xoff,
                                             (uint32_t)((i >> 2) * 128 + (i & 3) * 32) * 2u, 0, 0);

  // 2. Weight ring prologue.
  const int tl = active ? tile0 : 0;
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(reinterpret_cast<const char*>(wfrag) + (size_t)tl * GP * kBlockBytes, (uint32_t)(RF * GP * kBlockBytes));
  const uint32_t woff = (uint32_t)lane * 16u;
  const uint32_t sboff = kSbOffsetBytes + (uint32_t)tok * 8u;
  const int last = GP - 1;
  WStage<RF> ws[NS];
  if (active) {
#pragma unroll
    for (int p = 0; p < NS; ++p) load_w<RF>(ws[p], rw, woff, sboff, min(p, last), GP);
  }
  // 3. The slab is complete once every wave's DMA has landed.
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");

  f32x4_t acc[RF];
#pragma unroll
  for (int r = 0; r < RF; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (!active) return;
  const bf16x8_t ones = ones_operand();
  auto xfrag = [&](int gp) {
    XStage xs;
#pragma unroll
    for (int jh = 0; jh < 4; ++jh) xs.a[jh >> 1][jh & 1] = __builtin_bit_cast(bf16x8_t, slab[(gp * 4 + jh) * 64 + lane]);
    return xs;
  };
  int base = 0;
  for (; base + NS < GP; base += NS) {
#pragma unroll
    for (int p = 0; p < NS; ++p) {
      compute<RF>(xfrag(base + p), ws[p], acc, ones);
      load_w<RF>(ws[p], rw, woff, sboff, min(base + p + NS, last), GP);
      __builtin_amdgcn_sched_barrier(0);  // ring order, as in the wave-X kernel
    }
  }
#pragma unroll
  for (int p = 0; p < NS; ++p)
    if (base + p < GP) compute<RF>(xfrag(base + p), ws[p], acc, ones);

  // 4. Output. Lane (col, quad) holds tokens 4*quad + i of row col of each of its tiles.
  const int col = tok;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = quad * 4 + i;
    if (t >= M) continue;
    if constexpr (EPI == kSwiGlu) {
      const float g = bf16_bits_to_f32(f32_to_bf16_bits(acc[0][i]));
      const float u = bf16_bits_to_f32(f32_to_bf16_bits(acc[1][i]));
      y[(size_t)t * ldy + (size_t)(tile0 >> 1) * 16 + col] = silu_mul_bf16(g, u);
    } else {
#pragma unroll
      for (int r = 0; r < RF; ++r) {
        const size_t c = EPI == kGluSplit ? (size_t)r * (N >> 1) + (size_t)(tile0 >> 1) * 16 + col
                                          : (size_t)(tile0 + r) * 16 + col;
        y[(size_t)t * ldy + c] = f32_to_bf16_bits(acc[r][i]);
      }
    }
  }
}

using WaveXKernel = void (*)(const uint16_t*, int, int, int, const uint32_t*, int, int, uint16_t*, int, const EpiArgs);

// 16-wave workgroups cap a wave at 128 VGPRs; ring depths that would spill there are left out.
constexpr int kMaxNs16[5] = {0, 4, 3, 0, 0};
// Eight-wave workgroups cap a wave at 256 VGPRs; four-tile rings deeper than 3 would not fit.
constexpr int kMaxNsRf4 = 3;

// The conv and split-K epilogues are built for the ring depths and wave counts the decoder
// shapes use (ns <= 4, waves <= 8), which keeps the number of kernel instances in check.
constexpr bool compact_epilogue(int e) { return e >= kConv; }

template <int RF, int NS, int EPI>
WaveXKernel wavex_sk(int sk) {
  switch (sk) {
    case 1: return qmm_wavex_kernel<RF, 1, NS, EPI>;
    case 2: return qmm_wavex_kernel<RF, 2, NS, EPI>;
    case 4: return qmm_wavex_kernel<RF, 4, NS, EPI>;
    case 8: return qmm_wavex_kernel<RF, 8, NS, EPI>;
    case 16:
      if constexpr (NS <= kMaxNs16[RF] && !compact_epilogue(EPI)) return qmm_wavex_kernel<RF, 16, NS, EPI>;
      return nullptr;
    default: return nullptr;
  }
}

template <int NS, int EPI>
WaveXKernel wavex_rf(int rf, int sk) {
  if constexpr (EPI == kGluSplit || EPI == kSwiGlu) {
    return rf == 2 ? wavex_sk<2, NS, EPI>(sk) : nullptr;
  } else {
    switch (rf) {
      case 1: return wavex_sk<1, NS, EPI>(sk);
      case 2: return wavex_sk<2, NS, EPI>(sk);
      case 4:
        if constexpr (NS <= kMaxNsRf4) return wavex_sk<4, NS, EPI>(sk);
        return nullptr;
      default: return nullptr;
    }
  }
}

template <int EPI>
WaveXKernel pick_wavex(int rf, int sk, int ns) {
  switch (ns) {
    case 2: return wavex_rf<2, EPI>(rf, sk);
    case 3: return wavex_rf<3, EPI>(rf, sk);
    case 4: return wavex_rf<4, EPI>(rf, sk);
    case 5:
      if constexpr (!compact_epilogue(EPI) || EPI == kConv) return wavex_rf<5, EPI>(rf, sk);
      return nullptr;
    default: return nullptr;
  }
}

template <int RF, int EPI>
WaveXKernel slab_ns(int ns) {
  switch (ns) {
    case 2: return qmm_slab_kernel<RF, 2, EPI>;
    case 3: return qmm_slab_kernel<RF, 3, EPI>;
    case 4: return qmm_slab_kernel<RF, 4, EPI>;
    case 6:
      if constexpr (RF <= 2) return qmm_slab_kernel<RF, 6, EPI>;
      return nullptr;
    case 8:
      if constexpr (RF == 1) return qmm_slab_kernel<RF, 8, EPI>;
      return nullptr;
    default: return nullptr;
  }
}

template <int EPI>
WaveXKernel pick_slab(int rf, int ns) {
  if constexpr (EPI >= kPartial) {
    return nullptr;  // split-K and conv epilogues use wave-X tiles only
  } else if constexpr (EPI != kPlain) {
    return rf == 2 ? slab_ns<2, EPI>(ns) : nullptr;
  } else {
    switch (rf) {
      case 1: return slab_ns<1, EPI>(ns);
      case 2: return slab_ns<2, EPI>(ns);
      case 4: return slab_ns<4, EPI>(ns);
      default: return nullptr;
    }
  }
}

// The slab holds 4 KB of X fragments per group pair (16 token rows x 128 k of bf16).
constexpr size_t kSlabBytesPerPair = 4096;
constexpr size_t kMaxSlabBytes = 96 * 1024;

// kSplitK instances: rf 1, 2 (4 to 16 waves, rings of 2 to 4) and 4 (4 or 8 waves, rings of 2 or 3).
template <int RF, int NS>
WaveXKernel splitk_sk(int sk) {
  switch (sk) {
    case 4: return qmm_wavex_kernel<RF, 4, NS, kSplitK>;
    case 8: return qmm_wavex_kernel<RF, 8, NS, kSplitK>;
    case 16:
      if constexpr (NS <= kMaxNs16[RF]) return qmm_wavex_kernel<RF, 16, NS, kSplitK>;
      return nullptr;
    default: return nullptr;
  }
}

template <int NS>
WaveXKernel splitk_rf(int rf, int sk) {
  switch (rf) {
    case 1: return splitk_sk<1, NS>(sk);
    case 2: return splitk_sk<2, NS>(sk);
    case 4:
      if constexpr (NS <= kMaxNsRf4) return sk <= 8 ? splitk_sk<4, NS>(sk) : nullptr;
      return nullptr;
    default: return nullptr;
  }
}

WaveXKernel pick_splitk(const skinny_qmm_tile& t) {
  if (t.kind != SKINNY_QMM_WAVE_X) return nullptr;
  switch (t.ns) {
    case 2: return splitk_rf<2>(t.rf, t.waves);
    case 3: return splitk_rf<3>(t.rf, t.waves);
    case 4: return splitk_rf<4>(t.rf, t.waves);
    default: return nullptr;
  }
}

template <int EPI>
WaveXKernel pick_kernel(const skinny_qmm_tile& t) {
  if constexpr (EPI == kSplitK) return pick_splitk(t);
  return t.kind == SKINNY_QMM_SLAB_X ? pick_slab<EPI>(t.rf, t.ns) : pick_wavex<EPI>(t.rf, t.waves, t.ns);
}

// One-wave forms of multi-wave tiles: the tile's K groups accumulated in one wave (wavex_body's
// VS), bitwise the tile's products. Taken from kOneWaveMinM tokens on: for the 36-layer decoders'
// gate|up the 4-wave tile is the faster one for a single token (with the RMSNorm formed inside
// it), the one-wave form from two tokens on.
constexpr int kOneWaveMinM = 2;

template <int EPI>
WaveXKernel one_wave_form(const skinny_qmm_tile& t, int K, int splits) {
  if constexpr (EPI == kSwiGlu) {
    // four groups of five pairs: K = 2560 in one split
    if (t.kind == SKINNY_QMM_WAVE_X && t.rf == 2 && t.waves == 4 && t.ns == 2 && K == 20 * 128 && splits == 1)
      return qmm_wavex_kernel<2, 1, 4, kSwiGlu, false, false, 4, 5>;
  }
  return nullptr;
}

// Enqueues the tile's kernel for epilogue EPI over N output rows (the caller checked the tile).
template <int EPI>
int launch_tile(const skinny_qmm_tile& t, const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N,
                uint16_t* y, int ldy, void* stream, int splits = 1, const EpiArgs& ea = EpiArgs{}) {
  const WaveXKernel kern = pick_kernel<EPI>(t);
  if (!kern) return skinny_set_error(SKINNY_EINVAL, "qmm: no kernel for tile kind=%d rf=%d waves=%d ns=%d", t.kind, t.rf,
                                     t.waves, t.ns);
  const int groups = (N / 16) / t.rf;
  if (const WaveXKernel one = M >= kOneWaveMinM ? one_wave_form<EPI>(t, K, splits) : nullptr) {
    hipLaunchKernelGGL(one, dim3(groups, splits), dim3(64), 0, (hipStream_t)stream, x, M, K, ldx, w_frag, N, splits, y,
                       ldy, ea);
    return skinny_check_launch("qmm");
  }
  if (t.kind == SKINNY_QMM_WAVE_X) {
    hipLaunchKernelGGL(kern, dim3(groups, splits), dim3(64 * t.waves), 0, (hipStream_t)stream, x, M, K, ldx, w_frag, N, splits,
                       y, ldy, ea);
    return skinny_check_launch("qmm");
  }
  const size_t lds = (size_t)(K / 128) * kSlabBytesPerPair;
  if (lds > 64 * 1024) {
    // Dynamic LDS beyond 64 KB must be allowed per kernel once; repeating the call is harmless.
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return skinny_set_error(SKINNY_ELAUNCH, "qmm: slab of %zu bytes: %s", lds, hipGetErrorString(e));
  }
  hipLaunchKernelGGL(kern, dim3((groups + t.waves - 1) / t.waves), dim3(64 * t.waves), lds, (hipStream_t)stream, x, M,
                     K, ldx, w_frag, N, 1, y, ldy, ea);
  return skinny_check_launch("qmm");
}

// Gated-norm-in instances: the split-K tiles of the decoders' Gated-DeltaNet out_proj (the 36-layer
// hybrid's 2048 x 2560 and the test decoder's 256 x 256).
WaveXKernel pick_gated(const skinny_qmm_tile& t) {
  if (t.kind != SKINNY_QMM_WAVE_X) return nullptr;
  switch (t.rf * 1000 + t.waves * 10 + t.ns) {
    case 2043: return qmm_wavex_kernel<2, 4, 3, kPartial, false, true>;
    case 1022: return qmm_wavex_kernel<1, 2, 2, kPartial, false, true>;
    default: return nullptr;
  }
}

// Norm-in instances: the tiles the decoders' RMSNorm consumers take (the fused q|k|v, gate|up and
// Gated-DeltaNet input projections of the 36-layer and the test decoders).
template <int EPI>
WaveXKernel pick_normin(const skinny_qmm_tile& t) {
  if (t.kind != SKINNY_QMM_WAVE_X) return nullptr;
  const int key = t.rf * 1000 + t.waves * 10 + t.ns;
  if constexpr (EPI == kPlain) {
    switch (key) {
      case 2043: return qmm_wavex_kernel<2, 4, 3, kPlain, true>;
      case 1022: return qmm_wavex_kernel<1, 2, 2, kPlain, true>;
      default: return nullptr;
    }
  } else if constexpr (EPI == kSwiGlu) {
    switch (key) {
      case 2014: return qmm_wavex_kernel<2, 1, 4, kSwiGlu, true>;
      case 2022: return qmm_wavex_kernel<2, 2, 2, kSwiGlu, true>;
      case 2023: return qmm_wavex_kernel<2, 2, 3, kSwiGlu, true>;
      case 2024: return qmm_wavex_kernel<2, 2, 4, kSwiGlu, true>;
      case 2042: return qmm_wavex_kernel<2, 4, 2, kSwiGlu, true>;
      case 2043: return qmm_wavex_kernel<2, 4, 3, kSwiGlu, true>;
      case 2044: return qmm_wavex_kernel<2, 4, 4, kSwiGlu, true>;
      case 2082: return qmm_wavex_kernel<2, 8, 2, kSwiGlu, true>;
      default: return nullptr;
    }
  } else if constexpr (EPI == kConv) {
    switch (key) {
      // A 4-deep ring for the tile's 5 (the depth changes no bits): with 5 the norm-in instance
      // takes 254 VGPRs and 56 AGPRs, one wave per SIMD, and the 257th workgroup of a 2560 x 8224
      // projection runs after the others; with 4 it takes 254 VGPRs, two waves per SIMD.
      case 2045: return qmm_wavex_kernel<2, 4, 4, kConv, true>;
      default: return nullptr;
    }
  }
  return nullptr;
}

// Checks a tile against (K, N); returns 0 or an error code with the message set.
int check_tile(const skinny_qmm_tile& t, int K, int N) {
  const int GP = K / 128, T = N / 16;
  SKINNY_CHECK_ARG(t.kind == SKINNY_QMM_WAVE_X || t.kind == SKINNY_QMM_SLAB_X, "qmm tile: unknown kind %d", t.kind);
  SKINNY_CHECK_ARG(t.rf == 1 || t.rf == 2 || t.rf == 4, "qmm tile: rf=%d must be 1, 2 or 4", t.rf);
  SKINNY_CHECK_ARG(T % t.rf == 0, "qmm tile: N/16=%d not divisible by rf=%d", T, t.rf);
  if (t.kind == SKINNY_QMM_WAVE_X) {
    SKINNY_CHECK_ARG(t.waves >= 1 && t.waves <= GP, "qmm tile: waves=%d must be in [1, K/128=%d]", t.waves, GP);
  } else {
    SKINNY_CHECK_ARG(t.waves >= 1 && t.waves <= 8, "qmm tile: slab waves=%d must be in [1, 8]", t.waves);
    SKINNY_CHECK_ARG((size_t)GP * kSlabBytesPerPair <= kMaxSlabBytes, "qmm tile: K=%d too large for the X slab", K);
  }
  SKINNY_CHECK_ARG(pick_kernel<kPlain>(t) != nullptr, "qmm tile: unsupported tile kind=%d rf=%d waves=%d ns=%d",
                   t.kind, t.rf, t.waves, t.ns);
  return SKINNY_OK;
}

}  // namespace

static int launch_pack(bool forward, const uint32_t* w_mlx, const uint16_t* scales, const uint16_t* biases,
                       const uint32_t* w_frag, int N, int K, void* stream, const char* what) {
  SKINNY_CHECK_ARG(w_mlx && scales && biases && w_frag, "%s: null pointer", what);
  SKINNY_CHECK_ARG(N > 0 && N % 16 == 0, "%s: N=%d must be a positive multiple of 16", what, N);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0, "%s: K=%d must be a positive multiple of 128", what, K);
  SKINNY_CHECK_ARG(skinny_aligned(w_mlx, 4) && skinny_aligned(w_frag, 16) && skinny_aligned(scales, 2) &&
                       skinny_aligned(biases, 2),
                   "%s: misaligned buffer", what);
  SKINNY_CHECK_ARG((const void*)w_mlx != (const void*)w_frag, "%s: in-place is not supported", what);
  const size_t total = (size_t)(N / 16) * (K / 128) * kBlockWords;
  const int threads = 256;
  const size_t blocks = (total + threads - 1) / threads;
  const int grid = (int)(blocks < 65536 ? blocks : 65536);
  auto kern = forward ? pack_kernel<true> : pack_kernel<false>;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(threads), 0, (hipStream_t)stream, const_cast<uint32_t*>(w_mlx),
                     const_cast<uint16_t*>(scales), const_cast<uint16_t*>(biases), const_cast<uint32_t*>(w_frag), N,
                     K);
  return skinny_check_launch(what);
}

extern "C" int skinny_w4g64_pack(const uint32_t* w_mlx, const uint16_t* scales, const uint16_t* biases,
                                 uint32_t* w_frag, int N, int K, void* stream) {
  return launch_pack(true, w_mlx, scales, biases, w_frag, N, K, stream, "pack");
}

extern "C" int skinny_w4g64_unpack(const uint32_t* w_frag, uint32_t* w_mlx, uint16_t* scales, uint16_t* biases,
                                   int N, int K, void* stream) {
  return launch_pack(false, w_mlx, scales, biases, w_frag, N, K, stream, "unpack");
}

static int check_relayout(const uint32_t* a, const uint32_t* b, int N, int K, const char* what) {
  SKINNY_CHECK_ARG(a && b, "%s: null pointer", what);
  SKINNY_CHECK_ARG(N > 0 && N % 16 == 0, "%s: N=%d must be a positive multiple of 16", what, N);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0, "%s: K=%d must be a positive multiple of 128", what, K);
  SKINNY_CHECK_ARG(skinny_aligned(a, 16) && skinny_aligned(b, 16), "%s: buffers must be 16-byte aligned", what);
  SKINNY_CHECK_ARG((const void*)a != (const void*)b, "%s: in-place is not supported", what);
  return SKINNY_OK;
}

static int grid_for(size_t total) {
  const size_t blocks = (total + 255) / 256;
  return (int)(blocks < 65536 ? blocks : 65536);
}

extern "C" int skinny_w4g64_relayout(const uint32_t* w_mlx, uint32_t* w_frag, int N, int K, void* stream) {
  if (int rc = check_relayout(w_mlx, w_frag, N, K, "relayout")) return rc;
  hipLaunchKernelGGL((pack_kernel<true, 256>), dim3(grid_for((size_t)N * K / 8)), dim3(256), 0, (hipStream_t)stream,
                     const_cast<uint32_t*>(w_mlx), nullptr, nullptr, w_frag, N, K);
  return skinny_check_launch("relayout");
}

extern "C" int skinny_w4g64_unrelayout(const uint32_t* w_frag, uint32_t* w_mlx, int N, int K, void* stream) {
  if (int rc = check_relayout(w_frag, w_mlx, N, K, "unrelayout")) return rc;
  hipLaunchKernelGGL((pack_kernel<false, 256>), dim3(grid_for((size_t)N * K / 8)), dim3(256), 0, (hipStream_t)stream,
                     w_mlx, nullptr, nullptr, const_cast<uint32_t*>(w_frag), N, K);
  return skinny_check_launch("unrelayout");
}

extern "C" int skinny_w4g64_attach(const uint32_t* w_frag, const uint16_t* scales, const uint16_t* biases,
                                   uint32_t* packed, int N, int K, void* stream) {
  if (int rc = check_relayout(w_frag, packed, N, K, "attach")) return rc;
  SKINNY_CHECK_ARG(scales && biases && skinny_aligned(scales, 2) && skinny_aligned(biases, 2),
                   "attach: scales and biases must be non-null bf16 buffers");
  hipLaunchKernelGGL(attach_kernel, dim3(grid_for((size_t)(N / 16) * (K / 128) * kBlockWords)), dim3(256), 0,
                     (hipStream_t)stream, w_frag, scales, biases, packed, N, K);
  return skinny_check_launch("attach");
}

// Measured on MI355X at M = 1, 8 and 16 (rotating weight sets larger than the 256 MB Infinity
// Cache, launches captured in a HIP graph): the tile with the smallest summed time over the three
// M per (K, N) of the decoder workloads. {K, N, kind, rf, waves, ns}.
constexpr int kTileTable[][6] = {
    {2560, 6144, SKINNY_QMM_WAVE_X, 2, 4, 3},    // fused q|k|v
    {4096, 2560, SKINNY_QMM_WAVE_X, 1, 8, 2},    // o_proj
    {2560, 19456, SKINNY_QMM_WAVE_X, 2, 2, 2},   // fused gate|up
    {9728, 2560, SKINNY_QMM_WAVE_X, 1, 8, 2},    // down
    {2560, 151936, SKINNY_QMM_SLAB_X, 1, 8, 4},  // lm_head
    {2560, 9728, SKINNY_QMM_WAVE_X, 4, 4, 2},    // single matmul of the headline shape
    {2560, 8224, SKINNY_QMM_WAVE_X, 2, 4, 5},    // fused Gated-DeltaNet q|k|v|z|b|a
    {2560, 32768, SKINNY_QMM_WAVE_X, 4, 4, 2},   // pruned draft head (first 32768 rows of lm_head)
    // Qwen3.5-4B's projections (16 gated q heads + 4 kv heads of dim 256; Gated-DeltaNet with 16
    // key and 32 value heads of dim 128), measured inside that decoder's verify step at M = 1, 8, 16.
    {2560, 10240, SKINNY_QMM_WAVE_X, 4, 2, 2},   // fused q|gate|k|v
    {2560, 12352, SKINNY_QMM_WAVE_X, 4, 4, 3},   // fused Gated-DeltaNet q|k|v|z|b|a (conv epilogue)
    {2560, 248320, SKINNY_QMM_SLAB_X, 2, 8, 4},  // lm_head (vocabulary 248320): 75 against 80 us at M=16
};

extern "C" int skinny_qmm_pick_tile(int K, int N, skinny_qmm_tile* tile) {
  SKINNY_CHECK_ARG(tile, "pick_tile: null output");
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && N > 0 && N % 16 == 0, "pick_tile: bad shape K=%d N=%d", K, N);
  for (const auto& e : kTileTable)
    if (e[0] == K && e[1] == N) {
      *tile = skinny_qmm_tile{e[2], e[3], e[4], e[5]};
      return SKINNY_OK;
    }
  // Other shapes: more row tiles per wave as N grows (X fragments shared by more rows); waves
  // per workgroup: the fewest that put >= 1024 waves in flight, at most one per group pair;
  // a 2-deep ring.
  const int GP = K / 128;
  const int tiles = N / 16;
  int r = 1;
  if (tiles >= 4096 && tiles % 4 == 0) r = 4;
  else if (tiles >= 384 && tiles % 2 == 0) r = 2;
  const int blocks = tiles / r;
  int s = 1;
  while (s < (r == 4 ? 8 : 16) && 2 * s <= GP && (long)blocks * s < 1024) s *= 2;
  *tile = skinny_qmm_tile{SKINNY_QMM_WAVE_X, r, s, 2};
  return SKINNY_OK;
}

extern "C" int skinny_qmm_w4g64_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N,
                                     uint16_t* y, int ldy, const skinny_qmm_tile* tile, void* stream) {
  SKINNY_CHECK_ARG(x && w_frag && y, "qmm: null pointer");
  SKINNY_CHECK_ARG(M >= 1 && M <= 16, "qmm: M=%d must be in [1, 16]", M);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0, "qmm: K=%d must be a positive multiple of 128", K);
  SKINNY_CHECK_ARG(N > 0 && N % 16 == 0, "qmm: N=%d must be a positive multiple of 16", N);
  SKINNY_CHECK_ARG(ldx >= K && ldx % 8 == 0, "qmm: ldx=%d must be >= K and a multiple of 8", ldx);
  SKINNY_CHECK_ARG(ldy >= N, "qmm: ldy=%d must be >= N", ldy);
  SKINNY_CHECK_ARG(skinny_aligned(x, 16), "qmm: x must be 16-byte aligned");
  SKINNY_CHECK_ARG(skinny_aligned(w_frag, 16), "qmm: w_frag must be 16-byte aligned");
  SKINNY_CHECK_ARG(skinny_aligned(y, 2), "qmm: y must be 2-byte aligned");
  SKINNY_CHECK_ARG((size_t)M * ldx * 2 < 0x40000000u, "qmm: x too large for a buffer descriptor");
  skinny_qmm_tile t;
  if (tile) {
    t = *tile;
  } else {
    int rc = skinny_qmm_pick_tile(K, N, &t);
    if (rc) return rc;
  }
  int rc = check_tile(t, K, N);
  if (rc) return rc;
  SKINNY_CHECK_ARG((size_t)t.rf * (K / 128) * kBlockBytes < 0x80000000u, "qmm: K too large for a buffer descriptor");
  return launch_tile<kPlain>(t, x, M, K, ldx, w_frag, N, y, ldy, stream);
}

extern "C" int skinny_qmm_w4g64_glu_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int F,
                                         uint16_t* y, int ldy, int swiglu, const skinny_qmm_tile* tile, void* stream) {
  SKINNY_CHECK_ARG(x && w_frag && y, "qmm glu: null pointer");
  SKINNY_CHECK_ARG(M >= 1 && M <= 16, "qmm glu: M=%d must be in [1, 16]", M);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0, "qmm glu: K=%d must be a positive multiple of 128", K);
  SKINNY_CHECK_ARG(F > 0 && F % 16 == 0, "qmm glu: F=%d must be a positive multiple of 16", F);
  SKINNY_CHECK_ARG(swiglu == 0 || swiglu == 1, "qmm glu: swiglu=%d must be 0 or 1", swiglu);
  SKINNY_CHECK_ARG(ldx >= K && ldx % 8 == 0, "qmm glu: ldx=%d must be >= K and a multiple of 8", ldx);
  SKINNY_CHECK_ARG(ldy >= (swiglu ? F : 2 * F), "qmm glu: ldy=%d too small", ldy);
  SKINNY_CHECK_ARG(skinny_aligned(x, 16) && skinny_aligned(w_frag, 16) && skinny_aligned(y, 2),
                   "qmm glu: misaligned buffer");
  SKINNY_CHECK_ARG((size_t)M * ldx * 2 < 0x40000000u, "qmm glu: x too large for a buffer descriptor");
  skinny_qmm_tile t;
  if (tile) {
    t = *tile;
  } else {
    int rc = skinny_qmm_glu_pick_tile(K, F, &t);
    if (rc) return rc;
  }
  SKINNY_CHECK_ARG(t.rf == 2, "qmm glu: the gate|up layout needs rf=2 (got %d)", t.rf);
  int rc = check_tile(t, K, 2 * F);
  if (rc) return rc;
  SKINNY_CHECK_ARG((size_t)2 * (K / 128) * kBlockBytes < 0x80000000u, "qmm glu: K too large for a buffer descriptor");
  return swiglu ? launch_tile<kSwiGlu>(t, x, M, K, ldx, w_frag, 2 * F, y, ldy, stream)
                : launch_tile<kGluSplit>(t, x, M, K, ldx, w_frag, 2 * F, y, ldy, stream);
}

// Split-K tiles of the projections whose output only feeds a residual RMSNorm (skinny_rmsnorm_
// partials_bf16 or a norm-in matmul adds the slices), measured inside the decoder's verify step at
// M = 1, 8 and 16 (the step's X comes from memory, so isolated-matmul timings rank these
// differently).
// {K, N, splits, rf, waves, ns}.
constexpr int kPartialTable[][6] = {
    {9728, 2560, 3, 2, 4, 3},  // down
    {4096, 2560, 3, 2, 4, 3},  // o_proj
    {2048, 2560, 3, 2, 4, 3},  // Gated-DeltaNet out_proj
    {9216, 2560, 3, 2, 4, 3},  // Qwen3.5-4B's down
};
constexpr int kMaxSplits = 4;

extern "C" int skinny_qmm_partial_pick(int K, int N, int* splits, skinny_qmm_tile* tile) {
  SKINNY_CHECK_ARG(splits && tile, "partial pick: null output");
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && N > 0 && N % 16 == 0, "partial pick: bad shape K=%d N=%d", K, N);
  for (const auto& e : kPartialTable)
    if (e[0] == K && e[1] == N) {
      *splits = e[2];
      *tile = skinny_qmm_tile{SKINNY_QMM_WAVE_X, e[3], e[4], e[5]};
      return SKINNY_OK;
    }
  // Other shapes: the unsplit tile (a wave-X one), split until >= 256 workgroups or 4 splits,
  // while each split keeps a group pair per wave.
  int rc = skinny_qmm_pick_tile(K, N, tile);
  if (rc) return rc;
  if (tile->kind != SKINNY_QMM_WAVE_X) *tile = skinny_qmm_tile{SKINNY_QMM_WAVE_X, 2, 8, 2};
  if ((N / 16) % tile->rf) tile->rf = 1;
  const int groups = (N / 16) / tile->rf, GP = K / 128;
  int s = 1;
  while (2 * s <= kMaxSplits && groups * s < 256 && GP / (2 * s) >= tile->waves) s *= 2;
  while (GP / s < tile->waves) tile->waves /= 2;
  *splits = s;
  return SKINNY_OK;
}

extern "C" int skinny_qmm_w4g64_partial_f32(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N,
                                            float* part, int ldp, int splits, const skinny_qmm_tile* tile,
                                            void* stream) {
  SKINNY_CHECK_ARG(x && w_frag && part, "qmm partial: null pointer");
  SKINNY_CHECK_ARG(M >= 1 && M <= 16, "qmm partial: M=%d must be in [1, 16]", M);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0, "qmm partial: K=%d must be a positive multiple of 128", K);
  SKINNY_CHECK_ARG(N > 0 && N % 16 == 0, "qmm partial: N=%d must be a positive multiple of 16", N);
  SKINNY_CHECK_ARG(ldx >= K && ldx % 8 == 0, "qmm partial: ldx=%d must be >= K and a multiple of 8", ldx);
  SKINNY_CHECK_ARG(ldp >= N, "qmm partial: ldp=%d must be >= N", ldp);
  SKINNY_CHECK_ARG(splits >= 1 && splits <= kMaxSplits, "qmm partial: splits=%d must be in [1, %d]", splits,
                   kMaxSplits);
  SKINNY_CHECK_ARG(skinny_aligned(x, 16) && skinny_aligned(w_frag, 16) && skinny_aligned(part, 4),
                   "qmm partial: misaligned buffer");
  SKINNY_CHECK_ARG((size_t)M * ldx * 2 < 0x40000000u, "qmm partial: x too large for a buffer descriptor");
  skinny_qmm_tile t;
  if (tile) {
    t = *tile;
  } else {
    int s = 0;
    int rc = skinny_qmm_partial_pick(K, N, &s, &t);
    if (rc) return rc;
  }
  SKINNY_CHECK_ARG(t.kind == SKINNY_QMM_WAVE_X, "qmm partial: split-K needs a wave-X tile");
  int rc = check_tile(t, K, N);
  if (rc) return rc;
  SKINNY_CHECK_ARG((K / 128) / splits >= t.waves, "qmm partial: %d waves need >= %d group pairs per split (K=%d, %d splits)",
                   t.waves, t.waves, K, splits);
  SKINNY_CHECK_ARG((size_t)t.rf * (K / 128) * kBlockBytes < 0x80000000u, "qmm partial: K too large for a buffer descriptor");
  return launch_tile<kPartial>(t, x, M, K, ldx, w_frag, N, reinterpret_cast<uint16_t*>(part), ldp, stream, splits);
}

// Split-K plain tiles, measured on MI355X over rotating weight sets at M = 1, 8 and 16 (launches
// captured back to back in a HIP graph): {K, N, splits, rf, waves, ns}. Shapes not listed take the
// unsplit kernel (splits = 1).
constexpr int kSplitKTable[][6] = {
    {9728, 2560, 3, 2, 8, 3},  // the MLP down projection of the 36-layer decoders
};

extern "C" size_t skinny_qmm_splitk_workspace_bytes(int N, int splits) {
  if (N <= 0 || splits < 2) return 0;
  return kSplitKHeaderWords * sizeof(float) + (size_t)(splits - 1) * 16 * (size_t)N * sizeof(float);
}

extern "C" int skinny_qmm_splitk_pick(int K, int N, int* splits, skinny_qmm_tile* tile) {
  SKINNY_CHECK_ARG(splits && tile, "splitk pick: null output");
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && N > 0 && N % 16 == 0, "splitk pick: bad shape K=%d N=%d", K, N);
  for (const auto& e : kSplitKTable)
    if (e[0] == K && e[1] == N) {
      *splits = e[2];
      *tile = skinny_qmm_tile{SKINNY_QMM_WAVE_X, e[3], e[4], e[5]};
      return SKINNY_OK;
    }
  *splits = 1;
  return skinny_qmm_pick_tile(K, N, tile);
}

extern "C" int skinny_qmm_w4g64_splitk_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N,
                                            uint16_t* y, int ldy, float* workspace, size_t workspace_bytes, int splits,
                                            const skinny_qmm_tile* tile, void* stream) {
  SKINNY_CHECK_ARG(x && w_frag && y && workspace, "qmm splitk: null pointer");
  SKINNY_CHECK_ARG(M >= 1 && M <= 16, "qmm splitk: M=%d must be in [1, 16]", M);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0, "qmm splitk: K=%d must be a positive multiple of 128", K);
  SKINNY_CHECK_ARG(N > 0 && N % 16 == 0, "qmm splitk: N=%d must be a positive multiple of 16", N);
  SKINNY_CHECK_ARG(ldx >= K && ldx % 8 == 0, "qmm splitk: ldx=%d must be >= K and a multiple of 8", ldx);
  SKINNY_CHECK_ARG(ldy >= N, "qmm splitk: ldy=%d must be >= N", ldy);
  SKINNY_CHECK_ARG(splits >= 2 && splits <= kMaxSplitK, "qmm splitk: splits=%d must be in [2, %d]", splits, kMaxSplitK);
  SKINNY_CHECK_ARG(workspace_bytes >= skinny_qmm_splitk_workspace_bytes(N, splits),
                   "qmm splitk: workspace of %zu bytes, needs %zu", workspace_bytes,
                   skinny_qmm_splitk_workspace_bytes(N, splits));
  SKINNY_CHECK_ARG(skinny_aligned(x, 16) && skinny_aligned(w_frag, 16) && skinny_aligned(workspace, 16),
                   "qmm splitk: misaligned buffer");
  SKINNY_CHECK_ARG((size_t)M * ldx * 2 < 0x40000000u, "qmm splitk: x too large for a buffer descriptor");
  skinny_qmm_tile t;
  if (tile) {
    t = *tile;
  } else {
    int s = 0;
    if (int rc = skinny_qmm_splitk_pick(K, N, &s, &t)) return rc;
  }
  SKINNY_CHECK_ARG(t.kind == SKINNY_QMM_WAVE_X, "qmm splitk: needs a wave-X tile");
  if (int rc = check_tile(t, K, N)) return rc;
  SKINNY_CHECK_ARG(pick_splitk(t) != nullptr, "qmm splitk: no split-K kernel for rf=%d waves=%d ns=%d", t.rf, t.waves,
                   t.ns);
  SKINNY_CHECK_ARG((K / 128) / splits >= t.waves, "qmm splitk: %d waves need >= %d group pairs per split (K=%d, %d splits)",
                   t.waves, t.waves, K, splits);
  SKINNY_CHECK_ARG((size_t)t.rf * (K / 128) * kBlockBytes < 0x80000000u, "qmm splitk: K too large for a buffer descriptor");
  EpiArgs ea{};
  ea.part = workspace;
  return launch_tile<kSplitK>(t, x, M, K, ldx, w_frag, N, y, ldy, stream, splits, ea);
}

// Fused gate|up + SwiGLU tiles measured inside the decoder step (its X, the RMSNorm output just
// written, arrives from memory rather than from L2 as in a back-to-back matmul loop), over the
// verify step at M = 1, 8 and 16: {K, F, kind, rf, waves, ns}.
constexpr int kGluTileTable[][6] = {
    {2560, 9728, SKINNY_QMM_WAVE_X, 2, 4, 2},  // 36-layer decoders' MLP (one-wave form from 2 tokens on)
    {2560, 9216, SKINNY_QMM_WAVE_X, 2, 4, 2},  // Qwen3.5-4B's MLP (the same forms)
};

extern "C" int skinny_qmm_glu_pick_tile(int K, int F, skinny_qmm_tile* tile) {
  SKINNY_CHECK_ARG(F > 0 && F % 16 == 0, "glu pick_tile: F=%d must be a positive multiple of 16", F);
  SKINNY_CHECK_ARG(tile, "glu pick_tile: null output");
  for (const auto& e : kGluTileTable)
    if (e[0] == K && e[1] == F) {
      *tile = skinny_qmm_tile{e[2], e[3], e[4], e[5]};
      return SKINNY_OK;
    }
  int rc = skinny_qmm_pick_tile(K, 2 * F, tile);
  if (rc) return rc;
  if (tile->rf != 2) {  // the gate|up pairing fixes two row tiles per wave
    tile->rf = 2;
    if (pick_kernel<kPlain>(*tile) == nullptr) tile->ns = 2;
  }
  return SKINNY_OK;
}

// A wave-X tile within the wave counts and ring depths the compact epilogues are built for.
static skinny_qmm_tile wavex_tile(skinny_qmm_tile t, int K) {
  if (t.kind != SKINNY_QMM_WAVE_X) {
    int w = 8;
    while (w > 1 && w > K / 128) w >>= 1;
    t = skinny_qmm_tile{SKINNY_QMM_WAVE_X, t.rf, w, 2};
  }
  if (t.ns > 4) t.ns = 4;
  if (t.waves > 8) t.waves = 8;
  return t;
}

// ---------------------------------------------------------------------------------------------
// The Gated-DeltaNet input projection with the mixer's conv + SiLU in its epilogue.

// The conv epilogue's default tile: the plain one as a wave-X tile within the wave counts and ring
// depths the epilogue is built for.
static int conv_default_tile(int K, int N, skinny_qmm_tile* out) {
  skinny_qmm_tile t;
  int rc = skinny_qmm_pick_tile(K, N, &t);
  if (rc) return rc;
  t = wavex_tile(t, K);
  if (t.rf == 4 && t.ns > 3) t.ns = 3;
  if (t.kind == SKINNY_QMM_WAVE_X && t.ns == 4 && t.rf <= 2) {
    skinny_qmm_tile plain;
    if (skinny_qmm_pick_tile(K, N, &plain) == SKINNY_OK && plain.kind == SKINNY_QMM_WAVE_X && plain.ns == 5 &&
        plain.waves <= 8)
      t.ns = 5;  // the plain tile's ring depth where the epilogue has an instance of it
  }
  *out = t;
  return SKINNY_OK;
}

extern "C" int skinny_qmm_w4g64_conv_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N,
                                          uint16_t* y, int ldy, int C, uint16_t* conv_state, const uint16_t* conv_w,
                                          int KW, uint16_t* window, const int32_t* parent,
                                          const skinny_qmm_tile* tile, void* stream) {
  SKINNY_CHECK_ARG(x && w_frag && y && conv_state && conv_w, "qmm conv: null pointer");
  SKINNY_CHECK_ARG(M >= 1 && M <= kConvTokens, "qmm conv: M=%d must be in [1, %d]", M, kConvTokens);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && N > 0 && N % 16 == 0, "qmm conv: bad shape K=%d N=%d", K, N);
  SKINNY_CHECK_ARG(KW == kConvKW, "qmm conv: kernel width %d unsupported (only %d)", KW, kConvKW);
  SKINNY_CHECK_ARG(C >= 16 && C % 16 == 0 && C <= N, "qmm conv: C=%d must be a multiple of 16 in [16, N=%d]", C, N);
  SKINNY_CHECK_ARG(ldx >= K && ldx % 8 == 0 && ldy >= N, "qmm conv: bad strides ldx=%d ldy=%d", ldx, ldy);
  SKINNY_CHECK_ARG(!parent || window, "qmm conv: a draft tree needs the window buffer");
  SKINNY_CHECK_ARG(skinny_aligned(x, 16) && skinny_aligned(w_frag, 16) && skinny_aligned(y, 2) &&
                       skinny_aligned(conv_state, 4) && skinny_aligned(conv_w, 4),
                   "qmm conv: misaligned buffer");
  SKINNY_CHECK_ARG((size_t)M * ldx * 2 < 0x40000000u, "qmm conv: x too large for a buffer descriptor");
  skinny_qmm_tile t;
  if (tile) {
    t = *tile;
  } else if (int rc = conv_default_tile(K, N, &t)) {
    return rc;
  }
  SKINNY_CHECK_ARG(t.kind == SKINNY_QMM_WAVE_X, "qmm conv: needs a wave-X tile");
  int rc = check_tile(t, K, N);
  if (rc) return rc;
  SKINNY_CHECK_ARG((size_t)t.rf * (K / 128) * kBlockBytes < 0x80000000u, "qmm conv: K too large for a buffer descriptor");
  EpiArgs ea{};
  ea.conv_C = C;
  ea.conv_state = conv_state;
  ea.conv_w = conv_w;
  ea.window = window;
  ea.parent = parent;
  return launch_tile<kConv>(t, x, M, K, ldx, w_frag, N, y, ldy, stream, 1, ea);
}

// ---------------------------------------------------------------------------------------------
// Norm-in forms: the projection of rmsnorm(h + residual) * w formed inside the matmul.

// The tile a norm-in call of `kind` takes by default: the plain entry point's, so both give the
// same bits.
static int normin_default_tile(int kind, int K, int N, skinny_qmm_tile* t) {
  if (kind == SKINNY_NORMIN_PLAIN) return skinny_qmm_pick_tile(K, N, t);
  if (kind == SKINNY_NORMIN_SWIGLU) return skinny_qmm_glu_pick_tile(K, N / 2, t);
  if (kind == SKINNY_NORMIN_CONV) return conv_default_tile(K, N, t);
  return skinny_set_error(SKINNY_EINVAL, "normin: unknown kind %d", kind);
}

static WaveXKernel normin_kernel(int kind, const skinny_qmm_tile& t) {
  if (kind == SKINNY_NORMIN_PLAIN) return pick_normin<kPlain>(t);
  if (kind == SKINNY_NORMIN_SWIGLU) return pick_normin<kSwiGlu>(t);
  if (kind == SKINNY_NORMIN_CONV) return pick_normin<kConv>(t);
  return nullptr;
}

extern "C" int skinny_qmm_normin_supported(int kind, int M, int K, int N, int splits, const skinny_qmm_tile* tile) {
  skinny_qmm_tile t;
  if (M < 1 || M > kNormInMaxM || K <= 0 || K % 128 || K > 16 * kMaxNormInTiles || N <= 0 || N % 16 || splits < 0 ||
      splits > kMaxSplits)
    return 0;
  if (tile) {
    t = *tile;
  } else if (normin_default_tile(kind, K, N, &t) != SKINNY_OK) {
    return 0;
  }
  if (check_tile(t, K, N) != SKINNY_OK || normin_kernel(kind, t) == nullptr) return 0;
  return NormInLayout(M, K, splits).bytes <= kNormInMaxLds;
}

static int launch_normin(int kind, const skinny_norm_in* ni, int M, int K, const uint32_t* w_frag, int N, uint16_t* y,
                         int ldy, const skinny_qmm_tile* tile, EpiArgs ea, void* stream, const char* what) {
  SKINNY_CHECK_ARG(ni && ni->h && ni->weight && w_frag && y, "%s: null pointer", what);
  SKINNY_CHECK_ARG(M >= 1 && M <= kNormInMaxM, "%s: M=%d must be in [1, %d]", what, M, kNormInMaxM);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && K <= 16 * kMaxNormInTiles && N > 0 && N % 16 == 0,
                   "%s: bad shape K=%d (a multiple of 128, at most %d) N=%d", what, K, 16 * kMaxNormInTiles, N);
  SKINNY_CHECK_ARG(ni->splits >= 0 && ni->splits <= kMaxSplits && (ni->splits == 0) == (ni->parts == nullptr),
                   "%s: splits=%d must be in [0, %d], with slices exactly when > 0", what, ni->splits, kMaxSplits);
  SKINNY_CHECK_ARG(skinny_aligned(ni->h, 16) && skinny_aligned(ni->weight, 16) && skinny_aligned(w_frag, 16) &&
                       (!ni->parts || skinny_aligned(ni->parts, 16)) && (!ni->h_out || skinny_aligned(ni->h_out, 16)) &&
                       skinny_aligned(y, 2),
                   "%s: misaligned buffer", what);
  SKINNY_CHECK_ARG((const void*)ni->h_out != (const void*)ni->h, "%s: h_out must not alias h (every workgroup reads h)",
                   what);
  skinny_qmm_tile t;
  if (tile) {
    t = *tile;
  } else if (int rc = normin_default_tile(kind, K, N, &t)) {
    return rc;
  }
  if (int rc = check_tile(t, K, N)) return rc;
  const WaveXKernel kern = normin_kernel(kind, t);
  SKINNY_CHECK_ARG(kern != nullptr, "%s: no norm-in kernel for tile rf=%d waves=%d ns=%d", what, t.rf, t.waves, t.ns);
  const NormInLayout L(M, K, ni->splits);
  SKINNY_CHECK_ARG(L.bytes <= kNormInMaxLds, "%s: %u bytes of LDS for M=%d K=%d splits=%d exceed %u", what, L.bytes, M,
                   K, ni->splits, kNormInMaxLds);
  SKINNY_CHECK_ARG((size_t)ni->splits * M * K * 4 < 0x80000000u && (size_t)t.rf * (K / 128) * kBlockBytes < 0x80000000u,
                   "%s: too large for a buffer descriptor", what);
  if (L.bytes > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)L.bytes);
    if (e != hipSuccess) return skinny_set_error(SKINNY_ELAUNCH, "%s: LDS of %u bytes: %s", what, L.bytes, hipGetErrorString(e));
  }
  ea.ni_h = ni->h;
  ea.ni_parts = ni->parts;
  ea.ni_splits = ni->splits;
  ea.ni_w = ni->weight;
  ea.ni_eps = ni->eps;
  ea.ni_hout = ni->h_out;
  hipLaunchKernelGGL(kern, dim3((N / 16) / t.rf, 1), dim3(64 * t.waves), L.bytes, (hipStream_t)stream, nullptr, M, K, K,
                     w_frag, N, 1, y, ldy, ea);
  return skinny_check_launch(what);
}

extern "C" int skinny_qmm_w4g64_normin_bf16(const skinny_norm_in* ni, int M, int K, const uint32_t* w_frag, int N,
                                            uint16_t* y, int ldy, const skinny_qmm_tile* tile, void* stream) {
  SKINNY_CHECK_ARG(ldy >= N, "qmm normin: ldy=%d must be >= N=%d", ldy, N);
  return launch_normin(SKINNY_NORMIN_PLAIN, ni, M, K, w_frag, N, y, ldy, tile, EpiArgs{}, stream, "qmm normin");
}

extern "C" int skinny_qmm_w4g64_glu_normin_bf16(const skinny_norm_in* ni, int M, int K, const uint32_t* w_frag, int F,
                                                uint16_t* y, int ldy, const skinny_qmm_tile* tile, void* stream) {
  SKINNY_CHECK_ARG(F > 0 && F % 16 == 0 && ldy >= F, "qmm glu normin: F=%d (multiple of 16), ldy=%d >= F", F, ldy);
  SKINNY_CHECK_ARG(!tile || tile->rf == 2, "qmm glu normin: the gate|up layout needs rf=2");
  return launch_normin(SKINNY_NORMIN_SWIGLU, ni, M, K, w_frag, 2 * F, y, ldy, tile, EpiArgs{}, stream,
                       "qmm glu normin");
}

extern "C" int skinny_qmm_w4g64_conv_normin_bf16(const skinny_norm_in* ni, int M, int K, const uint32_t* w_frag, int N,
                                                 uint16_t* y, int ldy, int C, uint16_t* conv_state,
                                                 const uint16_t* conv_w, int KW, uint16_t* window,
                                                 const int32_t* parent, const skinny_qmm_tile* tile, void* stream) {
  SKINNY_CHECK_ARG(conv_state && conv_w, "qmm conv normin: null pointer");
  SKINNY_CHECK_ARG(KW == kConvKW, "qmm conv normin: kernel width %d unsupported (only %d)", KW, kConvKW);
  SKINNY_CHECK_ARG(C >= 16 && C % 16 == 0 && C <= N, "qmm conv normin: C=%d must be a multiple of 16 in [16, N=%d]", C,
                   N);
  SKINNY_CHECK_ARG(ldy >= N, "qmm conv normin: ldy=%d must be >= N=%d", ldy, N);
  SKINNY_CHECK_ARG(!parent || window, "qmm conv normin: a draft tree needs the window buffer");
  SKINNY_CHECK_ARG(skinny_aligned(conv_state, 4) && skinny_aligned(conv_w, 4), "qmm conv normin: misaligned buffer");
  EpiArgs ea{};
  ea.conv_C = C;
  ea.conv_state = conv_state;
  ea.conv_w = conv_w;
  ea.window = window;
  ea.parent = parent;
  return launch_normin(SKINNY_NORMIN_CONV, ni, M, K, w_frag, N, y, ldy, tile, ea, stream, "qmm conv normin");
}

// Workgroups of `kern` (256 threads, no dynamic LDS) the current device holds at once, looked up
// once per device.
static int resident_workgroups(const void* kern, int* out) {
  static std::mutex mu;
  static int cached[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return skinny_set_error(SKINNY_ELAUNCH, "qkv attention: hipGetDevice: %s", hipGetErrorString(e));
  SKINNY_CHECK_ARG(dev >= 0 && dev < 64, "qkv attention: device %d beyond 64", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (!cached[dev]) {
    int cus = 0, per_cu = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 64 * kWaves, 0);
    if (e != hipSuccess)
      return skinny_set_error(SKINNY_ELAUNCH, "qkv attention: occupancy query: %s", hipGetErrorString(e));
    cached[dev] = cus * per_cu;
  }
  *out = cached[dev];
  return SKINNY_OK;
}

extern "C" int skinny_qkv_attention_fused_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N,
                                               uint16_t* handoff, int ld_handoff, int Hq, int Hkv, int D,
                                               const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                               const float* rope_table, int rope_positions, const int32_t* pos0,
                                               const int32_t* tree, uint16_t* k_cache, uint16_t* vt_cache, int maxlen,
                                               float scale, float* workspace, size_t workspace_bytes, uint16_t* out,
                                               void* stream) {
  SKINNY_CHECK_ARG(x && w_frag && handoff && rope_table && pos0 && k_cache && vt_cache && workspace && out,
                   "qkv attention: null pointer");
  SKINNY_CHECK_ARG(D == kD, "qkv attention: head dim %d unsupported (only %d)", D, kD);
  SKINNY_CHECK_ARG(Hkv >= 1 && Hq % Hkv == 0 && N == (Hq + 2 * Hkv) * D,
                   "qkv attention: N=%d must be (Hq=%d + 2 Hkv=%d) x %d, Hq a multiple of Hkv", N, Hq, Hkv, D);
  SKINNY_CHECK_ARG(M >= 1 && M <= kFusedMaxTokens && (Hq / Hkv) * M <= kRowsMax,
                   "qkv attention: M=%d (at most %d) with %d query rows per kv head (at most %d)", M, kFusedMaxTokens,
                   (Hq / Hkv) * M, kRowsMax);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && ldx >= K && ldx % 8 == 0 && skinny_aligned(x, 16),
                   "qkv attention: K=%d (multiple of 128), ldx=%d (>= K, multiple of 8), x 16-byte aligned", K, ldx);
  SKINNY_CHECK_ARG(ld_handoff >= N && ld_handoff % 8 == 0 && skinny_aligned(handoff, 16),
                   "qkv attention: ld_handoff=%d (>= N, multiple of 8), hand-off buffer 16-byte aligned", ld_handoff);
  SKINNY_CHECK_ARG(maxlen >= kChunk && maxlen % kChunk == 0 && rope_positions >= maxlen,
                   "qkv attention: maxlen=%d must be a multiple of %d and within the RoPE table (%d)", maxlen, kChunk,
                   rope_positions);
  SKINNY_CHECK_ARG(workspace_bytes >= skinny_attn_workspace_bytes(Hkv, maxlen), "qkv attention: workspace too small");
  SKINNY_CHECK_ARG(skinny_aligned(w_frag, 16) && skinny_aligned(k_cache, 16) && skinny_aligned(vt_cache, 16) &&
                       skinny_aligned(rope_table, 16) && (!q_norm || skinny_aligned(q_norm, 16)),
                   "qkv attention: weights, caches, table and q_norm must be 16-byte aligned");
  skinny_qmm_tile t;
  if (int rc = skinny_qmm_pick_tile(K, N, &t)) return rc;
  const QkvAttnKernel kern = pick_qkv_attn(t);
  SKINNY_CHECK_ARG(kern, "qkv attention: no fused kernel for the (K=%d, N=%d) tile (rf=%d, waves=%d, ns=%d)", K, N,
                   t.rf, t.waves, t.ns);
  const int nch = maxlen / kChunk;
  const int n_proj = (N / 16) / t.rf;
  const int grid = n_proj + Hkv * nch;
  int resident = 0;
  if (int rc = resident_workgroups(reinterpret_cast<const void*>(kern), &resident)) return rc;
  SKINNY_CHECK_ARG(grid <= resident,
                   "qkv attention: %d workgroups (%d projection + %d x %d chunks) do not fit on the GPU at once (%d)", grid,
                   n_proj, Hkv, nch, resident);
  QkvAttnArgs aa{};
  aa.fa = FusedArgs{ld_handoff, q_norm, k_norm, eps, rope_table};
  aa.Hq = Hq;
  aa.Hkv = Hkv;
  aa.maxlen = maxlen;
  aa.nch = nch;
  aa.scale = scale;
  aa.kc = k_cache;
  aa.vt = vt_cache;
  aa.tree = tree;
  aa.part_o = workspace;
  aa.part_ml = workspace + (size_t)Hkv * nch * kRowsMax * kD;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kWaves), 0, (hipStream_t)stream, pos0, x, w_frag, handoff, M, K, ldx, N,
                     n_proj, aa);
  if (int rc = skinny_check_launch("qkv attention")) return rc;
  return attn_combine_launch(aa.part_o, aa.part_ml, M, Hq, Hkv, pos0, nch, out, reinterpret_cast<uint32_t*>(handoff),
                             ld_handoff / 2, N / 2, (hipStream_t)stream);
}

extern "C" int skinny_qkv_attention_supported(int K, int N, int Hkv, int maxlen) {
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && N > 0 && N % 16 == 0 && Hkv >= 1 && maxlen >= kChunk && maxlen % kChunk == 0,
                   "qkv attention supported: bad shape K=%d N=%d Hkv=%d maxlen=%d", K, N, Hkv, maxlen);
  skinny_qmm_tile t;
  if (int rc = skinny_qmm_pick_tile(K, N, &t)) return rc;
  const QkvAttnKernel kern = pick_qkv_attn(t);
  if (!kern) return 0;
  int resident = 0;
  if (int rc = resident_workgroups(reinterpret_cast<const void*>(kern), &resident)) return rc;
  return (N / 16) / t.rf + Hkv * (maxlen / kChunk) <= resident ? 1 : 0;
}

extern "C" int skinny_qmm_gated_partial_supported(int K, int N) {
  int splits = 0;
  skinny_qmm_tile t;
  if (skinny_qmm_partial_pick(K, N, &splits, &t) != SKINNY_OK) return 0;
  return pick_gated(t) != nullptr && (K / 128) / splits >= t.waves ? 1 : 0;
}

extern "C" int skinny_qmm_w4g64_gated_partial_f32(const float* y, int ldy, const uint16_t* z, int ldz,
                                                  const uint16_t* norm_w, float eps, int M, int K,
                                                  const uint32_t* w_frag, int N, float* part, int ldp, void* stream) {
  SKINNY_CHECK_ARG(y && z && norm_w && w_frag && part, "qmm gated partial: null pointer");
  SKINNY_CHECK_ARG(M >= 1 && M <= 16, "qmm gated partial: M=%d must be in [1, 16]", M);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && N > 0 && N % 16 == 0,
                   "qmm gated partial: K=%d (heads of 128), N=%d (multiple of 16)", K, N);
  SKINNY_CHECK_ARG(ldy >= K && ldy % 4 == 0 && ldz >= K && ldz % 8 == 0 && ldp >= N,
                   "qmm gated partial: ldy=%d (>= K, multiple of 4), ldz=%d (>= K, multiple of 8), ldp=%d (>= N)", ldy,
                   ldz, ldp);
  SKINNY_CHECK_ARG(skinny_aligned(y, 16) && skinny_aligned(z, 16) && skinny_aligned(norm_w, 16) &&
                       skinny_aligned(w_frag, 16) && skinny_aligned(part, 4),
                   "qmm gated partial: misaligned buffer");
  SKINNY_CHECK_ARG((size_t)M * ldy * 4 < 0x40000000u && (size_t)M * ldz * 2 < 0x40000000u,
                   "qmm gated partial: y or z too large for a buffer descriptor");
  int splits = 0;
  skinny_qmm_tile t;
  if (int rc = skinny_qmm_partial_pick(K, N, &splits, &t)) return rc;
  const WaveXKernel kern = pick_gated(t);
  SKINNY_CHECK_ARG(kern && (K / 128) / splits >= t.waves,
                   "qmm gated partial: no gated-norm-in kernel for the (K=%d, N=%d) split-K tile (rf=%d, waves=%d, ns=%d)",
                   K, N, t.rf, t.waves, t.ns);
  if (int rc = check_tile(t, K, N)) return rc;
  SKINNY_CHECK_ARG((size_t)t.rf * (K / 128) * kBlockBytes < 0x80000000u,
                   "qmm gated partial: K too large for a buffer descriptor");
  EpiArgs ea{};
  ea.gn_y = y;
  ea.gn_ldy = ldy;
  ea.gn_z = z;
  ea.gn_ldz = ldz;
  ea.gn_w = norm_w;
  ea.gn_eps = eps;
  hipLaunchKernelGGL(kern, dim3((N / 16) / t.rf, splits), dim3(64 * t.waves), 0, (hipStream_t)stream, nullptr, M, K, K,
                     w_frag, N, splits, reinterpret_cast<uint16_t*>(part), ldp, ea);
  return skinny_check_launch("qmm gated partial");
}

// --- the MLP sublayer in one launch -------------------------------------------------------------

namespace {

// The fused MLP launch's tiles: gate|up the one-wave form of the table's 4-group tile (K must be its
// 20 group pairs), down the partial table's (3 splits, rf 2, 4 waves, ring 3). 0 when (K, F, N) take
// them, else an error code with the message set.
int mlp_fused_check(int M, int K, int F, int N) {
  SKINNY_CHECK_ARG(M >= kOneWaveMinM && M <= 16, "mlp fused: M=%d must be in [%d, 16]", M, kOneWaveMinM);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && F > 0 && F % 128 == 0 && (F / 16) % kMlpProdTiles == 0 && N > 0 &&
                       N % 32 == 0,
                   "mlp fused: bad shape K=%d F=%d N=%d", K, F, N);
  skinny_qmm_tile g;
  if (int rc = skinny_qmm_glu_pick_tile(K, F, &g)) return rc;
  SKINNY_CHECK_ARG(one_wave_form<kSwiGlu>(g, K, 1) != nullptr,
                   "mlp fused: the gate|up tile for (K=%d, F=%d) has no one-wave form", K, F);
  int splits = 0;
  skinny_qmm_tile d;
  if (int rc = skinny_qmm_partial_pick(F, N, &splits, &d)) return rc;
  SKINNY_CHECK_ARG(splits == 3 && d.kind == SKINNY_QMM_WAVE_X && d.rf == 2 && d.waves == 4 && d.ns == 3,
                   "mlp fused: the down tile for (K=%d, N=%d) is not the fused launch's (3 splits, rf 2, 4 waves, ring 3)",
                   F, N);
  const int per_split = (F / 128 + splits - 1) / splits;
  SKINNY_CHECK_ARG((per_split + 3) / 4 <= 64 && per_split >= 4, "mlp fused: %d group pairs per split", per_split);
  return SKINNY_OK;
}

}  // namespace

extern "C" size_t skinny_mlp_fused_sync_bytes(int F) {
  if (F <= 0 || F % 128) return 0;
  return (size_t)(F / 128 + 1) * kSyncStride * sizeof(uint32_t);
}

extern "C" int skinny_mlp_fused_supported(int M, int K, int F, int N) {
  return mlp_fused_check(M, K, F, N) == SKINNY_OK ? 1 : 0;
}

extern "C" int skinny_mlp_fused_partial_f32(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_gate_up, int F,
                                            const uint32_t* w_down, int N, uint16_t* act, float* part,
                                            uint32_t* sync, size_t sync_bytes, void* stream) {
  SKINNY_CHECK_ARG(x && w_gate_up && w_down && act && part && sync, "mlp fused: null pointer");
  if (int rc = mlp_fused_check(M, K, F, N)) return rc;
  SKINNY_CHECK_ARG(ldx >= K && ldx % 8 == 0, "mlp fused: ldx=%d must be >= K and a multiple of 8", ldx);
  SKINNY_CHECK_ARG(sync_bytes >= skinny_mlp_fused_sync_bytes(F), "mlp fused: sync of %zu bytes, needs %zu", sync_bytes,
                   skinny_mlp_fused_sync_bytes(F));
  SKINNY_CHECK_ARG(skinny_aligned(x, 16) && skinny_aligned(w_gate_up, 16) && skinny_aligned(w_down, 16) &&
                       skinny_aligned(act, 16) && skinny_aligned(part, 4) && skinny_aligned(sync, 4),
                   "mlp fused: misaligned buffer");
  SKINNY_CHECK_ARG((size_t)M * ldx * 2 < 0x40000000u && (size_t)M * F * 2 < 0x40000000u,
                   "mlp fused: rows too large for a buffer descriptor");
  SKINNY_CHECK_ARG((size_t)2 * (K / 128) * kBlockBytes < 0x80000000u && (size_t)2 * (F / 128) * kBlockBytes < 0x80000000u,
                   "mlp fused: K too large for a buffer descriptor");
  const int n_prod = (F / 16) / kMlpProdTiles;
  const int consumers = (N / 32) * 3;
  EpiArgs ea{};
  ea.sync = sync;
  ea.sync_groups = F / 128;
  ea.sync_expect = 128 / 16;
  ea.sync_consumers = consumers;
  hipLaunchKernelGGL(mlp_fused_kernel, dim3(n_prod + consumers), dim3(256), 0, (hipStream_t)stream, x, M, K, ldx,
                     w_gate_up, F, w_down, N, 3, n_prod, act, part, ea);
  return skinny_check_launch("mlp fused");
}
