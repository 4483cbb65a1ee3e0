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
//    offset is wave-uniform (SGPR) and the lane part constant, so no address
//    arithmetic runs per stage. X rows past M use an out-of-range offset and read
//    as zeros without touching memory.
//  * Each wave owns RF row tiles x a contiguous group range, re-using one X
//    fragment across its RF tiles; SK waves of a workgroup split K and are
//    reduced through LDS in a fixed order. The tile depends on (K, N) only, so
//    a token's output is bitwise identical for every M.
#include "common.h"

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

template <bool kForward>
__global__ void pack_kernel(uint32_t* __restrict__ w_mlx, uint16_t* __restrict__ sc, uint16_t* __restrict__ bi,
                            uint32_t* __restrict__ frag, int N, int K) {
  const int G = K >> 6, GP = K >> 7, KW = K >> 3;
  const size_t total = (size_t)(N >> 4) * GP * kBlockWords;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int wi = (int)(i % kBlockWords);
    const size_t blk = i / kBlockWords;
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

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
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

// RF row tiles per wave; SK waves per workgroup split the K/128 group pairs as evenly as
// possible (wave w owns [w*GP/SK, (w+1)*GP/SK)). Each wave streams its pairs through a ring
// of NS stages; a stage holds one pair's weights, scales, biases AND X fragments, issued
// together NS pairs ahead of use. The pair consumed next is therefore always the oldest
// outstanding load, which is what the in-order vmcnt counter can wait for without stalling
// on younger prefetches. Refill rounds have no control flow around loads; loads past the
// wave's last pair repeat that pair (cache hits) and are not consumed.
template <int RF, int SK, int NS>
__global__ __launch_bounds__(64 * SK) void qmm_w4g64_kernel(const uint16_t* __restrict__ x, int M, int K, int ldx,
                                                            const uint32_t* __restrict__ wfrag, int N,
                                                            uint16_t* __restrict__ y, int ldy) {
  const int GP = K >> 7;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tile0 = blockIdx.x * RF;
  const int tok = lane & 15;
  const int quad = lane >> 4;
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(reinterpret_cast<const char*>(wfrag) + (size_t)tile0 * GP * kBlockBytes, (uint32_t)(RF * GP * kBlockBytes));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((size_t)M * ldx * 2));
  const uint32_t xoff = tok < M ? (uint32_t)(tok * ldx + quad * 8) * 2u : 0x40000000u;
  const uint32_t woff = (uint32_t)lane * 16u;
  const uint32_t sboff = kSbOffsetBytes + (uint32_t)tok * 8u;
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

  const int gpa = wave * GP / SK;
  const int npairs = (wave + 1) * GP / SK - gpa;  // >= 1: the host keeps sk <= K/128
  const int last = gpa + npairs - 1;

  WStage<RF> ws[NS];
  XStage xs[NS];
#pragma unroll
  for (int p = 0; p < NS; ++p) {
    const int gp = min(gpa + p, last);
    load_w<RF>(ws[p], rw, woff, sboff, gp, GP);
    load_x(xs[p], rx, xoff, gp);
  }

  f32x4_t acc[RF];
#pragma unroll
  for (int r = 0; r < RF; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  int base = 0;
  for (; base + NS < npairs; base += NS) {  // rounds that refill the ring
#pragma unroll
    for (int p = 0; p < NS; ++p) {
      compute<RF>(xs[p], ws[p], acc, ones);
      const int gp = min(gpa + base + p + NS, last);
      load_w<RF>(ws[p], rw, woff, sboff, gp, GP);
      load_x(xs[p], rx, xoff, gp);
    }
  }
#pragma unroll
  for (int p = 0; p < NS; ++p)  // final round: 1..NS pairs left, all in the ring
    if (base + p < npairs) compute<RF>(xs[p], ws[p], acc, ones);

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

using QmmKernel = void (*)(const uint16_t*, int, int, int, const uint32_t*, int, uint16_t*, int);

// 16-wave workgroups cap a wave at 128 VGPRs; ring depths that would spill there are left out.
constexpr int kMaxNs16[3] = {0, 4, 3};

template <int RF, int NS>
QmmKernel pick_sk(int sk) {
  switch (sk) {
    case 1: return qmm_w4g64_kernel<RF, 1, NS>;
    case 2: return qmm_w4g64_kernel<RF, 2, NS>;
    case 4: return qmm_w4g64_kernel<RF, 4, NS>;
    case 8: return qmm_w4g64_kernel<RF, 8, NS>;
    case 16: return NS <= kMaxNs16[RF] ? qmm_w4g64_kernel<RF, 16, NS> : nullptr;
    default: return nullptr;
  }
}

template <int NS>
QmmKernel pick_rf(int rf, int sk) {
  switch (rf) {
    case 1: return pick_sk<1, NS>(sk);
    case 2: return pick_sk<2, NS>(sk);
    default: return nullptr;
  }
}

// ns: ring depth (group pairs in flight per wave).
QmmKernel pick_kernel(int rf, int sk, int ns) {
  switch (ns) {
    case 2: return pick_rf<2>(rf, sk);
    case 3: return pick_rf<3>(rf, sk);
    case 4: return pick_rf<4>(rf, sk);
    case 5: return pick_rf<5>(rf, sk);
    default: return nullptr;
  }
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

extern "C" int skinny_qmm_pick_tile(int K, int N, int* rf, int* sk, int* ns) {
  SKINNY_CHECK_ARG(rf && sk && ns, "pick_tile: null output");
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0 && N > 0 && N % 16 == 0, "pick_tile: bad shape K=%d N=%d", K, N);
  const int GP = K / 128;
  const int tiles = N / 16;
  // Two row tiles per wave once there are enough tiles to keep the chip busy (X fragments are
  // then shared by 32 rows); waves per workgroup: the fewest that put >= 1024 waves in flight,
  // at most one per group pair; a 2-deep ring. From a sweep of the decoder shapes on MI355X.
  // Keyed by (K, N) only.
  const int r = (tiles >= 384 && tiles % 2 == 0) ? 2 : 1;
  const int blocks = tiles / r;
  int s = 1;
  while (s < 16 && 2 * s <= GP && (long)blocks * s < 1024) s *= 2;
  *rf = r;
  *sk = s;
  *ns = 2;
  return SKINNY_OK;
}

extern "C" int skinny_qmm_w4g64_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N,
                                     uint16_t* y, int ldy, int rf, int sk, int ns, void* stream) {
  SKINNY_CHECK_ARG(x && w_frag && y, "qmm: null pointer");
  SKINNY_CHECK_ARG(M >= 1 && M <= 16, "qmm: M=%d must be in [1, 16]", M);
  SKINNY_CHECK_ARG(K > 0 && K % 128 == 0, "qmm: K=%d must be a positive multiple of 128", K);
  SKINNY_CHECK_ARG(N > 0 && N % 16 == 0, "qmm: N=%d must be a positive multiple of 16", N);
  SKINNY_CHECK_ARG(ldx >= K && ldx % 8 == 0, "qmm: ldx=%d must be >= K and a multiple of 8", ldx);
  SKINNY_CHECK_ARG(ldy >= N, "qmm: ldy=%d must be >= N", ldy);
  SKINNY_CHECK_ARG(skinny_aligned(x, 16), "qmm: x must be 16-byte aligned");
  SKINNY_CHECK_ARG(skinny_aligned(w_frag, 16), "qmm: w_frag must be 16-byte aligned");
  SKINNY_CHECK_ARG(skinny_aligned(y, 2), "qmm: y must be 2-byte aligned");
  if (rf == 0 && sk == 0 && ns == 0) {
    int rc = skinny_qmm_pick_tile(K, N, &rf, &sk, &ns);
    if (rc) return rc;
  }
  const int GP = K / 128;
  SKINNY_CHECK_ARG(sk >= 1 && sk <= GP, "qmm: sk=%d must be in [1, K/128=%d]", sk, GP);
  QmmKernel kern = pick_kernel(rf, sk, ns);
  SKINNY_CHECK_ARG(kern != nullptr, "qmm: unsupported tile rf=%d sk=%d ns=%d", rf, sk, ns);
  SKINNY_CHECK_ARG((N / 16) % rf == 0, "qmm: N/16=%d not divisible by rf=%d", N / 16, rf);
  SKINNY_CHECK_ARG((size_t)M * ldx * 2 < 0x40000000u, "qmm: x too large for a buffer descriptor");
  SKINNY_CHECK_ARG((size_t)rf * (K / 128) * kBlockBytes < 0x80000000u, "qmm: K too large for a buffer descriptor");
  const int grid = (N / 16) / rf;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * sk), 0, (hipStream_t)stream, x, M, K, ldx, w_frag, N, y, ldy);
  return skinny_check_launch("qmm");
}
