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
//  * Nibbles are fed to the MFMA raw: (w & 0x000F000F) | 0x43004300 is a pair of
//    bf16 values 128+q (exact), so the group result is
//      s * (G - 128*xs) + b * xs  =  s * G + (b - 128 s) * xs,
//    with G = sum x (128+q) and xs = sum x, both from MFMA (xs against a ones
//    operand, which lands directly in the accumulator lane layout).
//  * Weights are relaid once into fragment order (skinny_w4g64_relayout): one
//    64-bit word per lane per (16-row tile, group), so each wave load is 512
//    contiguous bytes and the lane's two words are exactly its two B operands.
//  * Each wave owns RF row tiles x a contiguous group range, re-using one X
//    fragment across its RF tiles; SK waves of a workgroup split K and are
//    reduced through LDS in a fixed order. The tile depends on (K, N) only, so
//    a token's output is bitwise identical for every M.
#include "common.h"

namespace {

constexpr uint32_t kNibMask = 0x000F000Fu;
constexpr uint32_t kBf16Base = 0x43004300u;  // bf16 128.0 in both halves

// One MLX word (elements e0..e7 at bits 4e) -> fragment word (e_{2i} at 4i, e_{2i+1} at 16+4i).
__host__ __device__ __forceinline__ uint32_t mlx_to_frag_word(uint32_t w) {
  uint32_t o = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o |= ((w >> (8 * i)) & 0xFu) << (4 * i);
    o |= ((w >> (8 * i + 4)) & 0xFu) << (16 + 4 * i);
  }
  return o;
}

__host__ __device__ __forceinline__ uint32_t frag_to_mlx_word(uint32_t o) {
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w |= ((o >> (4 * i)) & 0xFu) << (8 * i);
    w |= ((o >> (16 + 4 * i)) & 0xFu) << (8 * i + 4);
  }
  return w;
}

// Fragment index of (tile t, group g, lane l) in u32x2 units.
__device__ __forceinline__ size_t frag_index(int t, int g, int l, int G) {
  return ((size_t)t * G + g) * 64 + l;
}

template <bool kForward>
__global__ void relayout_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, int N, int K) {
  const int G = K >> 6;
  const int KW = K >> 3;  // MLX words per row
  const size_t total = (size_t)(N >> 4) * G * 64;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63);
    const size_t tg = i >> 6;
    const int g = (int)(tg % G);
    const int t = (int)(tg / G);
    const int row = t * 16 + (l & 15);
    const int quad = l >> 4;
    const size_t w0 = (size_t)row * KW + g * 8 + quad;  // half 0: columns 64g + 8quad
    const size_t w1 = w0 + 4;                            // half 1: columns 64g + 32 + 8quad
    if (kForward) {
      u32x2_t o;
      o.x = mlx_to_frag_word(src[w0]);
      o.y = mlx_to_frag_word(src[w1]);
      reinterpret_cast<u32x2_t*>(dst)[i] = o;
    } else {
      const u32x2_t o = reinterpret_cast<const u32x2_t*>(src)[i];
      dst[w0] = frag_to_mlx_word(o.x);
      dst[w1] = frag_to_mlx_word(o.y);
    }
  }
}

__device__ __forceinline__ bf16x8_t unpack_nibbles(uint32_t w) {
  u32x4_t p;
  p.x = (w & kNibMask) | kBf16Base;
  p.y = ((w >> 4) & kNibMask) | kBf16Base;
  p.z = ((w >> 8) & kNibMask) | kBf16Base;
  p.w = ((w >> 12) & kNibMask) | kBf16Base;
  return __builtin_bit_cast(bf16x8_t, p);
}

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Per-group operands a wave keeps in flight.
template <int RF>
struct Stage {
  bf16x8_t a0, a1;        // X fragments, k 0..31 and 32..63 of the group
  u32x2_t w[RF];          // fragment words, one per row tile
  uint32_t s[RF], b[RF];  // bf16 bits of scale / bias for the lane's row
};

template <int RF>
__device__ __forceinline__ void load_stage(Stage<RF>& st, const bf16x8_t* __restrict__ xrow, bool has_tok, int quad,
                                           const u32x2_t* __restrict__ wf, const uint16_t* __restrict__ sc,
                                           const uint16_t* __restrict__ bi, int tile0, int g, int G, int lane,
                                           int nrow) {
  if (has_tok) {
    st.a0 = xrow[g * 8 + quad];
    st.a1 = xrow[g * 8 + 4 + quad];
  } else {
    st.a0 = bf16x8_t{};
    st.a1 = bf16x8_t{};
  }
#pragma unroll
  for (int r = 0; r < RF; ++r) {
    st.w[r] = wf[frag_index(tile0 + r, g, lane, G)];
    const size_t srow = (size_t)((tile0 + r) * 16 + nrow) * G + g;
    st.s[r] = sc[srow];
    st.b[r] = bi[srow];
  }
}

template <int RF>
__device__ __forceinline__ void compute_stage(const Stage<RF>& st, f32x4_t (&acc)[RF], const bf16x8_t ones) {
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  f32x4_t xs = mfma16x16x32(st.a0, ones, zero);
  xs = mfma16x16x32(st.a1, ones, xs);
#pragma unroll
  for (int r = 0; r < RF; ++r) {
    f32x4_t gacc = mfma16x16x32(st.a0, unpack_nibbles(st.w[r].x), zero);
    gacc = mfma16x16x32(st.a1, unpack_nibbles(st.w[r].y), gacc);
    const float s = bf16_bits_to_f32(st.s[r]);
    const float bp = fmaf(-128.0f, s, bf16_bits_to_f32(st.b[r]));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[r][j] = fmaf(s, gacc[j], acc[r][j]);
      acc[r][j] = fmaf(bp, xs[j], acc[r][j]);
    }
  }
}

constexpr int kUnroll = 4;  // groups whose loads are issued together

template <int RF, int SK>
__global__ __launch_bounds__(64 * SK) void qmm_w4g64_kernel(const uint16_t* __restrict__ x, int M, int K, int ldx,
                                                            const uint32_t* __restrict__ wfrag,
                                                            const uint16_t* __restrict__ sc,
                                                            const uint16_t* __restrict__ bi, int N,
                                                            uint16_t* __restrict__ y, int ldy, int GW) {
  const int G = K >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tile0 = blockIdx.x * RF;
  const int tok = lane & 15;
  const int quad = lane >> 4;
  const bool has_tok = tok < M;
  const bf16x8_t* xrow = reinterpret_cast<const bf16x8_t*>(x + (size_t)(has_tok ? tok : 0) * ldx);
  const u32x2_t* wf = reinterpret_cast<const u32x2_t*>(wfrag);
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

  f32x4_t acc[RF];
#pragma unroll
  for (int r = 0; r < RF; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int g_begin = wave * GW;
  const int g_end = g_begin + GW;
  int g = g_begin;
  for (; g + kUnroll <= g_end; g += kUnroll) {
    Stage<RF> st[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) load_stage<RF>(st[u], xrow, has_tok, quad, wf, sc, bi, tile0, g + u, G, lane, tok);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) compute_stage<RF>(st[u], acc, ones);
  }
  for (; g < g_end; ++g) {
    Stage<RF> st;
    load_stage<RF>(st, xrow, has_tok, quad, wf, sc, bi, tile0, g, G, lane, tok);
    compute_stage<RF>(st, acc, ones);
  }

  // Split-K reduction across the SK waves, in wave order.
  __shared__ float red[SK][RF][4][64];
#pragma unroll
  for (int r = 0; r < RF; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][r][j][lane] = acc[r][j];
  __syncthreads();
  // Output element (token t, tile r, row n) with n fastest so stores run along rows.
  for (int idx = threadIdx.x; idx < 16 * RF * 16; idx += 64 * SK) {
    const int n = idx & 15;
    const int r = (idx >> 4) % RF;
    const int t = idx / (16 * RF);
    if (t >= M) break;  // idx grows with t
    const int l = (t >> 2) * 16 + n;
    const int j = t & 3;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < SK; ++w) v += red[w][r][j][l];
    y[(size_t)t * ldy + (size_t)(tile0 + r) * 16 + n] = f32_to_bf16_bits(v);
  }
}

using QmmKernel = void (*)(const uint16_t*, int, int, int, const uint32_t*, const uint16_t*, const uint16_t*, int,
                           uint16_t*, int, int);

template <int RF>
QmmKernel pick_sk(int sk) {
  switch (sk) {
    case 1: return qmm_w4g64_kernel<RF, 1>;
    case 2: return qmm_w4g64_kernel<RF, 2>;
    case 4: return qmm_w4g64_kernel<RF, 4>;
    case 8: return qmm_w4g64_kernel<RF, 8>;
    case 16: return RF < 4 ? qmm_w4g64_kernel<RF, 16> : nullptr;  // RF=4 x 1024 threads spills
    default: return nullptr;
  }
}

QmmKernel pick_kernel(int rf, int sk) {
  switch (rf) {
    case 1: return pick_sk<1>(sk);
    case 2: return pick_sk<2>(sk);
    case 4: return pick_sk<4>(sk);
    default: return nullptr;
  }
}

}  // namespace

extern "C" int skinny_w4g64_relayout(const uint32_t* w_mlx, uint32_t* w_frag, int N, int K, void* stream) {
  SKINNY_CHECK_ARG(w_mlx && w_frag, "relayout: null pointer");
  SKINNY_CHECK_ARG(N > 0 && N % 16 == 0, "relayout: N=%d must be a positive multiple of 16", N);
  SKINNY_CHECK_ARG(K > 0 && K % 64 == 0, "relayout: K=%d must be a positive multiple of 64", K);
  SKINNY_CHECK_ARG(skinny_aligned(w_mlx, 4) && skinny_aligned(w_frag, 8), "relayout: misaligned buffer");
  SKINNY_CHECK_ARG((const void*)w_mlx != (const void*)w_frag, "relayout: in-place is not supported");
  const size_t total = (size_t)(N / 16) * (K / 64) * 64;
  const int threads = 256;
  const size_t blocks = (total + threads - 1) / threads;
  const int grid = (int)(blocks < 65536 ? blocks : 65536);
  hipLaunchKernelGGL(relayout_kernel<true>, dim3(grid), dim3(threads), 0, (hipStream_t)stream, w_mlx, w_frag, N, K);
  return skinny_check_launch("relayout");
}

extern "C" int skinny_w4g64_unrelayout(const uint32_t* w_frag, uint32_t* w_mlx, int N, int K, void* stream) {
  SKINNY_CHECK_ARG(w_mlx && w_frag, "unrelayout: null pointer");
  SKINNY_CHECK_ARG(N > 0 && N % 16 == 0, "unrelayout: N=%d must be a positive multiple of 16", N);
  SKINNY_CHECK_ARG(K > 0 && K % 64 == 0, "unrelayout: K=%d must be a positive multiple of 64", K);
  SKINNY_CHECK_ARG(skinny_aligned(w_mlx, 4) && skinny_aligned(w_frag, 8), "unrelayout: misaligned buffer");
  SKINNY_CHECK_ARG((const void*)w_mlx != (const void*)w_frag, "unrelayout: in-place is not supported");
  const size_t total = (size_t)(N / 16) * (K / 64) * 64;
  const int threads = 256;
  const size_t blocks = (total + threads - 1) / threads;
  const int grid = (int)(blocks < 65536 ? blocks : 65536);
  hipLaunchKernelGGL(relayout_kernel<false>, dim3(grid), dim3(threads), 0, (hipStream_t)stream, w_frag, w_mlx, N, K);
  return skinny_check_launch("unrelayout");
}

extern "C" int skinny_qmm_pick_tile(int K, int N, int* rf, int* sk, int* ks) {
  SKINNY_CHECK_ARG(rf && sk && ks, "pick_tile: null output");
  SKINNY_CHECK_ARG(K > 0 && K % 64 == 0 && N > 0 && N % 16 == 0, "pick_tile: bad shape K=%d N=%d", K, N);
  const int G = K / 64;
  const int tiles = N / 16;
  int r = (tiles >= 512 && tiles % 2 == 0) ? 2 : 1;
  const int blocks = tiles / r;
  // Smallest split of K (waves per workgroup) that puts >= 2048 waves in flight,
  // keeping >= 4 groups per wave; the table depends on (K, N) only.
  int s = 1;
  for (int cand = 1; cand <= 16; cand *= 2) {
    if (G % cand != 0 || G / cand < 4) break;
    s = cand;
    if ((long)blocks * cand >= 2048) break;
  }
  *rf = r;
  *sk = s;
  *ks = 1;
  return SKINNY_OK;
}

extern "C" size_t skinny_qmm_workspace_bytes(int N, int rf, int sk, int ks) {
  (void)N;
  (void)rf;
  (void)sk;
  (void)ks;
  return 0;
}

extern "C" int skinny_qmm_w4g64_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag,
                                     const uint16_t* scales, const uint16_t* biases, int N, uint16_t* y, int ldy,
                                     int rf, int sk, int ks, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  SKINNY_CHECK_ARG(x && w_frag && scales && biases && y, "qmm: null pointer");
  SKINNY_CHECK_ARG(M >= 1 && M <= 16, "qmm: M=%d must be in [1, 16]", M);
  SKINNY_CHECK_ARG(K > 0 && K % 64 == 0, "qmm: K=%d must be a positive multiple of 64", K);
  SKINNY_CHECK_ARG(N > 0 && N % 16 == 0, "qmm: N=%d must be a positive multiple of 16", N);
  SKINNY_CHECK_ARG(ldx >= K && ldx % 8 == 0, "qmm: ldx=%d must be >= K and a multiple of 8", ldx);
  SKINNY_CHECK_ARG(ldy >= N, "qmm: ldy=%d must be >= N", ldy);
  SKINNY_CHECK_ARG(skinny_aligned(x, 16), "qmm: x must be 16-byte aligned");
  SKINNY_CHECK_ARG(skinny_aligned(w_frag, 8), "qmm: w_frag must be 8-byte aligned");
  SKINNY_CHECK_ARG(skinny_aligned(scales, 2) && skinny_aligned(biases, 2) && skinny_aligned(y, 2),
                   "qmm: scales/biases/y must be 2-byte aligned");
  if (rf == 0 && sk == 0 && ks == 0) {
    int rc = skinny_qmm_pick_tile(K, N, &rf, &sk, &ks);
    if (rc) return rc;
  }
  const int G = K / 64;
  SKINNY_CHECK_ARG(ks == 1, "qmm: ks=%d unsupported (only 1)", ks);
  QmmKernel kern = pick_kernel(rf, sk);
  SKINNY_CHECK_ARG(kern != nullptr, "qmm: unsupported tile rf=%d sk=%d", rf, sk);
  SKINNY_CHECK_ARG((N / 16) % rf == 0, "qmm: N/16=%d not divisible by rf=%d", N / 16, rf);
  SKINNY_CHECK_ARG(G % sk == 0, "qmm: K/64=%d not divisible by sk=%d", G, sk);
  const int GW = G / sk;
  const int grid = (N / 16) / rf;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * sk), 0, (hipStream_t)stream, x, M, K, ldx, w_frag, scales, biases, N,
                     y, ldy, GW);
  return skinny_check_launch("qmm");
}
