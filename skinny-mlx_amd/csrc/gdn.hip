// Gated-DeltaNet pieces of the hybrid verify step and its replay-free rollback.
//
// Reference behaviour: mlx_lm's gated_delta_update as hooked by skinny_mlx/rollback.py:16,
// 39-42 (recurrence S <- g S (I - b k k^T) + b v k^T, y = S q; bench/reversal_check.py:5,
// 21-25, 43-47), the GDN short causal conv whose input rollback.py:44-52 records, and the
// rollback itself (rollback.py:58-73). The reference rolls back by re-running the recurrence
// over the accepted prefix; here the verify pass stores every per-token state S_1..S_M in HBM
// and rollback selects S_keep and the conv window on the device (no replay).
//
// State layout per layer: [H][Dv][Dk] fp32 (column j of S over Dk is contiguous), so the 16
// lanes that own one column read and write 512 contiguous bytes per token.
#include "common.h"

namespace {

constexpr int kDk = 128, kDv = 128;
constexpr int kCols = 8;   // value columns per workgroup (H x 16 workgroups)
constexpr int kPart = 16;  // lanes per column (8 key dims each)

__device__ __forceinline__ float sum16(float v) { return row16_sum(v); }

__device__ __forceinline__ float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }

// A draft tree's record of one layer (fp32 words), the operands of each node's state update as the
// tree pass forms them, for a node capacity of kTokBlock: the normalised q (scaled) and k of every
// node and head [T][H][2][Dk], then the decay and beta [T][H][2], then the v rows as bf16 [T][H*Dv].
struct GdnRecord {
  size_t qk, g, v, words;
  __host__ __device__ GdnRecord(int T, int H)
      : qk(0), g((size_t)T * H * 2 * kDk), v(g + (size_t)T * H * 2), words(v + (size_t)T * H * kDv / 2) {}
};

// Causal depthwise conv (kernel KW) over [conv_state (KW-1 rows); x (M rows)], then SiLU.
// One thread per channel. Tokens go in blocks of kTokBlock whose inputs are all loaded at once
// (one memory round trip per block); the thread writes the outputs, moves the last KW-1 rows into
// conv_state and, when `window` is set, keeps all M+KW-1 rows for rollback.
//
// Draft tree (`parent` set, M <= kTokBlock): node t's window is its own input and its ancestors'
// (parent pointers), running into the conv state above the root. The inputs and the state rows
// are staged in LDS (row KW-1+a for node a, rows 0..KW-2 the state) and in `window`; the conv
// state itself is left for the commit. The taps accumulate oldest first, as in the chain, so a
// chain-shaped tree is bitwise a chain.
constexpr int kConvThreads = 256;
constexpr int kTokBlock = 16;  // tokens staged per pass (and the most a draft tree may hold)

template <int KW>
__global__ __launch_bounds__(kConvThreads) void conv_silu_kernel(const uint16_t* __restrict__ x, int ldx, int M, int C,
                                                                 uint16_t* conv_state, const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ out, int ldo,
                                                                 uint16_t* __restrict__ window,
                                                                 const int32_t* __restrict__ parent) {
  __shared__ int par[kTokBlock];
  __shared__ int anc[kTokBlock][KW];  // tree: staged row of node t's tap j
  __shared__ uint16_t win[(KW - 1 + kTokBlock) * kConvThreads];  // tree: [row][thread]
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const bool own = c < C;
  float wv[KW];
  uint16_t hist[KW - 1];
  uint16_t xv[kTokBlock];  // the first block's inputs, loaded before the tree set-up below
#pragma unroll
  for (int j = 0; j < KW; ++j) wv[j] = own ? bf16_bits_to_f32(w[(size_t)c * KW + j]) : 0.f;
#pragma unroll
  for (int j = 0; j < KW - 1; ++j) hist[j] = own ? conv_state[(size_t)j * C + c] : (uint16_t)0;
#pragma unroll
  for (int i = 0; i < kTokBlock; ++i) xv[i] = own && i < M ? x[(size_t)i * ldx + c] : (uint16_t)0;
  if (parent) {
    if ((int)threadIdx.x < M) par[threadIdx.x] = parent[threadIdx.x];
    __syncthreads();
    if ((int)threadIdx.x < M) {  // tap j of node t: the input KW-1-j steps back along the ancestors
      int a = threadIdx.x;
#pragma unroll
      for (int j = KW - 1; j >= 0; --j) {
        anc[threadIdx.x][j] = KW - 1 + a;
        a = a >= 0 ? par[a] : a - 1;
      }
    }
    __syncthreads();
  }
  if (!own) return;
  if (window) {
#pragma unroll
    for (int j = 0; j < KW - 1; ++j) window[(size_t)j * C + c] = hist[j];
  }
  for (int t0 = 0; t0 < M; t0 += kTokBlock) {
    const int mb = min(kTokBlock, M - t0);
    if (t0 > 0) {
#pragma unroll
      for (int i = 0; i < kTokBlock; ++i) xv[i] = i < mb ? x[(size_t)(t0 + i) * ldx + c] : (uint16_t)0;
    }
    if (window) {
#pragma unroll
      for (int i = 0; i < kTokBlock; ++i)
        if (i < mb) window[(size_t)(KW - 1 + t0 + i) * C + c] = xv[i];
    }
    if (parent) {
      uint16_t* mine = win + threadIdx.x;
#pragma unroll
      for (int j = 0; j < KW - 1; ++j) mine[j * kConvThreads] = hist[j];
#pragma unroll
      for (int i = 0; i < kTokBlock; ++i)
        if (i < mb) mine[(KW - 1 + i) * kConvThreads] = xv[i];
#pragma unroll
      for (int t = 0; t < kTokBlock; ++t) {
        if (t >= mb) break;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < KW; ++j) acc = fmaf(wv[j], bf16_bits_to_f32(mine[anc[t][j] * kConvThreads]), acc);
        out[(size_t)t * ldo + c] = f32_to_bf16_bits(acc / (1.0f + expf(-acc)));
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < kTokBlock; ++i) {
      if (i >= mb) break;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < KW - 1; ++j) acc = fmaf(wv[j], bf16_bits_to_f32(hist[j]), acc);
      acc = fmaf(wv[KW - 1], bf16_bits_to_f32(xv[i]), acc);
      out[(size_t)(t0 + i) * ldo + c] = f32_to_bf16_bits(acc / (1.0f + expf(-acc)));
#pragma unroll
      for (int j = 0; j < KW - 2; ++j) hist[j] = hist[j + 1];
      hist[KW - 2] = xv[i];
    }
  }
#pragma unroll
  for (int j = 0; j < KW - 1; ++j) conv_state[(size_t)j * C + c] = hist[j];
}

// One token of the gated delta rule for the 8 key dims a lane holds of one value column (the
// column's 16 lanes together hold all 128): S <- decay S + k delta with delta = beta (v - k.(decay
// S)), then y = q.S. k.S is formed on the undecayed state and scaled once (decay (k.S)), in four
// partial sums, and so is q.S: short dependency chains, since the tokens run one after another.
// Returns y (the same in all 16 lanes of the column).
__device__ __forceinline__ float gdn_token(float (&s)[8], const float (&kh)[8], const float (&qh)[8], float v,
                                           float decay, float beta) {
  float a0 = s[0] * kh[0], a1 = s[1] * kh[1], a2 = s[2] * kh[2], a3 = s[3] * kh[3];
  a0 = fmaf(s[4], kh[4], a0);
  a1 = fmaf(s[5], kh[5], a1);
  a2 = fmaf(s[6], kh[6], a2);
  a3 = fmaf(s[7], kh[7], a3);
  const float delta = beta * (v - decay * sum16((a0 + a1) + (a2 + a3)));
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = fmaf(kh[e], delta, s[e] * decay);
  float b0 = s[0] * qh[0], b1 = s[1] * qh[1], b2 = s[2] * qh[2], b3 = s[3] * qh[3];
  b0 = fmaf(s[4], qh[4], b0);
  b1 = fmaf(s[5], qh[5], b1);
  b2 = fmaf(s[6], qh[6], b2);
  b3 = fmaf(s[7], qh[7], b3);
  return sum16((b0 + b1) + (b2 + b3));
}

template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

// Recurrence for one head h and value columns [kCols*blockIdx.y, +kCols): thread (column cc,
// part p) owns S[h][col][8p .. 8p+7]. qkv rows hold q | k | v, each H*Dk wide (v: H*Dv).
// Every block of kTokBlock tokens is staged first (q and k rows of head h, the workgroup's v
// columns, and each token's decay and beta gates: one memory round trip), then the normalised q
// and k of all its tokens are formed in parallel, so the sequential token loop is the state
// update alone, run from LDS. A draft tree's nodes
// keep their states in LDS (`snap`, dynamic) for their later children to continue from.
constexpr int kGdnThreads = kCols * kPart;

// kTree: the draft-tree form (parent pointers, per-node snapshots in LDS) is its own kernel, so
// the chain form carries none of its code (measured: 0.1-0.3 us faster per launch that way).
template <bool kTree>
__global__ __launch_bounds__(kGdnThreads) void gdn_kernel(const uint16_t* __restrict__ qkv, int ldq,
                                                          const uint16_t* __restrict__ bcol,
                                                          const uint16_t* __restrict__ acol, int ldab,
                                                          const float* __restrict__ A_log,
                                                          const float* __restrict__ dt_bias, float* state,
                                                          float* __restrict__ states_out, float* __restrict__ y,
                                                          const int32_t* __restrict__ parent, int M, int H,
                                                          float* __restrict__ record, int Hk) {
  __shared__ __attribute__((aligned(16))) uint16_t qk_lds[kTokBlock][2][kDk];
  __shared__ __attribute__((aligned(16))) float qkn_lds[kTokBlock][2][kDk];  // q * qn, k * kn
  __shared__ uint16_t v_lds[kTokBlock][kCols];
  __shared__ float gate_lds[kTokBlock][2];  // per token: decay, beta
  __shared__ int par_lds[kTokBlock];
  extern __shared__ f32x4_t snap[];  // draft tree: node t's state at [t][thread][2]
  const int h = blockIdx.x, tid = threadIdx.x;
  const int hk = h / (H / Hk);  // the key head this value head reads (q and k shared by H / Hk heads)
  const int cc = tid / kPart, p = tid % kPart;
  const int col = blockIdx.y * kCols + cc;
  const size_t sidx = ((size_t)h * kDv + col) * kDk + p * 8;
  float s[8];
  {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(state + sidx);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(state + sidx + 4);
    s[0] = a.x; s[1] = a.y; s[2] = a.z; s[3] = a.w; s[4] = b.x; s[5] = b.y; s[6] = b.z; s[7] = b.w;
  }
  const float neg_a = -expf(A_log[h]);
  const float dtb = dt_bias[h];
  const float qscale = rsqrtf((float)kDk);
  float s0[8];  // the state before the step: a draft tree's root and its restarts branch from it
#pragma unroll
  for (int e = 0; e < 8; ++e) s0[e] = s[e];
  for (int t0 = 0; t0 < M; t0 += kTokBlock) {
    const int mb = min(kTokBlock, M - t0);
    if (t0 > 0) __syncthreads();  // the previous block's staged rows are no longer read
    for (int i = tid; i < mb * 32; i += kGdnThreads) {  // q and k: 16 pieces of 16 bytes each per token
      const int t = i >> 5, sel = (i >> 4) & 1, piece = i & 15;
      *reinterpret_cast<u32x4_t*>(&qk_lds[t][sel][piece * 8]) = *reinterpret_cast<const u32x4_t*>(
          qkv + (size_t)(t0 + t) * ldq + (size_t)sel * Hk * kDk + (size_t)hk * kDk + piece * 8);
    }
    for (int i = tid; i < mb * kCols; i += kGdnThreads)
      v_lds[i / kCols][i % kCols] =
          qkv[(size_t)(t0 + i / kCols) * ldq + (size_t)2 * Hk * kDk + (size_t)h * kDv + blockIdx.y * kCols + i % kCols];
    if (tid < mb) {
      gate_lds[tid][0] = expf(neg_a * softplus(bf16_bits_to_f32(acol[(size_t)(t0 + tid) * ldab + h]) + dtb));
      gate_lds[tid][1] = 1.0f / (1.0f + expf(-bf16_bits_to_f32(bcol[(size_t)(t0 + tid) * ldab + h])));
      if constexpr (kTree) par_lds[tid] = parent[t0 + tid];
    }
    __syncthreads();
    // Normalised q and k of every token of the block, in parallel (they do not depend on the
    // state): 16-lane group g takes tokens g, g + kCols, ...; lane p its 8 dims.
    for (int i = cc; i < mb; i += kCols) {
      const u32x4_t qw = *reinterpret_cast<const u32x4_t*>(&qk_lds[i][0][p * 8]);
      const u32x4_t kw = *reinterpret_cast<const u32x4_t*>(&qk_lds[i][1][p * 8]);
      float q[8], k[8];
      float qq = 0.f, kk = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        q[e] = bf16_bits_to_f32((e & 1) ? (qw[e >> 1] >> 16) : (qw[e >> 1] & 0xffffu));
        k[e] = bf16_bits_to_f32((e & 1) ? (kw[e >> 1] >> 16) : (kw[e >> 1] & 0xffffu));
        qq = fmaf(q[e], q[e], qq);
        kk = fmaf(k[e], k[e], kk);
      }
      const float qn = rsqrtf(sum16(qq) + 1e-6f) * qscale;
      const float kn = rsqrtf(sum16(kk) + 1e-6f);
      f32x4_t* qd = reinterpret_cast<f32x4_t*>(&qkn_lds[i][0][p * 8]);
      f32x4_t* kd = reinterpret_cast<f32x4_t*>(&qkn_lds[i][1][p * 8]);
      qd[0] = f32x4_t{q[0] * qn, q[1] * qn, q[2] * qn, q[3] * qn};
      qd[1] = f32x4_t{q[4] * qn, q[5] * qn, q[6] * qn, q[7] * qn};
      kd[0] = f32x4_t{k[0] * kn, k[1] * kn, k[2] * kn, k[3] * kn};
      kd[1] = f32x4_t{k[4] * kn, k[5] * kn, k[6] * kn, k[7] * kn};
    }
    __syncthreads();
    if constexpr (kTree) {
      if (record) {  // the commit's replay operands (a tree is one block: t0 == 0)
        const GdnRecord rl(kTokBlock, H);
        if (blockIdx.y == 0) {  // this head's q, k and gates, once per head
          for (int i = tid; i < mb * 2 * kDk / 4; i += kGdnThreads) {
            const int t = i / (2 * kDk / 4), sel = (i / (kDk / 4)) & 1, piece = i % (kDk / 4);
            *reinterpret_cast<f32x4_t*>(record + rl.qk + (((size_t)t * H + h) * 2 + sel) * kDk + piece * 4) =
                *reinterpret_cast<const f32x4_t*>(&qkn_lds[t][sel][piece * 4]);
          }
          if (tid < mb) {
            record[rl.g + ((size_t)tid * H + h) * 2] = gate_lds[tid][0];
            record[rl.g + ((size_t)tid * H + h) * 2 + 1] = gate_lds[tid][1];
          }
        }
        uint16_t* rv = reinterpret_cast<uint16_t*>(record + rl.v);
        for (int i = tid; i < mb * kCols; i += kGdnThreads)
          rv[(size_t)(i / kCols) * H * kDv + (size_t)h * kDv + blockIdx.y * kCols + i % kCols] = v_lds[i / kCols][i % kCols];
      }
    }
    // Token i's operands from LDS.
    auto operands = [&](int i, float (&qh)[8], float (&kh)[8]) {
      const f32x4_t* qp = reinterpret_cast<const f32x4_t*>(&qkn_lds[i][0][p * 8]);
      const f32x4_t* kp = reinterpret_cast<const f32x4_t*>(&qkn_lds[i][1][p * 8]);
      const f32x4_t q0 = qp[0], q1 = qp[1], k0 = kp[0], k1 = kp[1];
      qh[0] = q0.x; qh[1] = q0.y; qh[2] = q0.z; qh[3] = q0.w; qh[4] = q1.x; qh[5] = q1.y; qh[6] = q1.z; qh[7] = q1.w;
      kh[0] = k0.x; kh[1] = k0.y; kh[2] = k0.z; kh[3] = k0.w; kh[4] = k1.x; kh[5] = k1.y; kh[6] = k1.z; kh[7] = k1.w;
    };
    // The token loops: no branches in their bodies (every lane of a column stores the column's y,
    // the same value to one address), two tokens per trip with two operand register sets, so token
    // i+1's operands come from LDS while token i computes.
    if constexpr (kTree) {
      // A draft tree: node t continues from the state before the step (no parent), from the state
      // just computed (parent t-1), or from its parent's snapshot, which an earlier trip wrote and
      // which is read ahead with the node's operands.
      struct Ops {
        float q[8], k[8], v, decay, beta;
        int pt;
        f32x4_t ps0, ps1;
      };
      auto fetch = [&](int i, Ops& o) {
        operands(i, o.q, o.k);
        o.v = bf16_bits_to_f32(v_lds[i][cc]);
        o.decay = gate_lds[i][0];
        o.beta = gate_lds[i][1];
        o.pt = par_lds[i];
        const size_t at = ((size_t)max(o.pt, 0) * kGdnThreads + tid) * 2;
        o.ps0 = snap[at];
        o.ps1 = snap[at + 1];
      };
      auto token = [&](int t, const Ops& o) {
        const float ps[8] = {o.ps0.x, o.ps0.y, o.ps0.z, o.ps0.w, o.ps1.x, o.ps1.y, o.ps1.z, o.ps1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] = o.pt < 0 ? s0[e] : (o.pt == t - 1 ? s[e] : ps[e]);
        const float yv = gdn_token(s, o.k, o.q, o.v, o.decay, o.beta);
        snap[((size_t)t * kGdnThreads + tid) * 2] = f32x4_t{s[0], s[1], s[2], s[3]};
        snap[((size_t)t * kGdnThreads + tid) * 2 + 1] = f32x4_t{s[4], s[5], s[6], s[7]};
        if (states_out) {  // a tree records its node states here or its operands in `record` (the entry point checks)
          float* dst = states_out + (size_t)t * H * kDv * kDk + sidx;
          *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{s[0], s[1], s[2], s[3]};
          *reinterpret_cast<f32x4_t*>(dst + 4) = f32x4_t{s[4], s[5], s[6], s[7]};
        }
        y[((size_t)t * H + h) * kDv + col] = yv;
      };
      Ops a, b;  // a tree is one block of at most kTokBlock nodes: t0 == 0
      fetch(0, a);
      int i = 0;
      for (; i + 1 < mb; i += 2) {
        fetch(i + 1, b);
        token(i, a);
        fetch(min(i + 2, mb - 1), a);
        token(i + 1, b);
      }
      if (i < mb) token(i, a);
    } else {
      auto chain = [&](auto record) {
        struct Ops {
          float q[8], k[8], v, decay, beta;
        };
        auto fetch = [&](int i, Ops& o) {
          operands(i, o.q, o.k);
          o.v = bf16_bits_to_f32(v_lds[i][cc]);
          o.decay = gate_lds[i][0];
          o.beta = gate_lds[i][1];
        };
        auto token = [&](int i, const Ops& o) {
          const int t = t0 + i;
          const float yv = gdn_token(s, o.k, o.q, o.v, o.decay, o.beta);
          if constexpr (decltype(record)::value) {
            float* dst = states_out + (size_t)t * H * kDv * kDk + sidx;
            *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{s[0], s[1], s[2], s[3]};
            *reinterpret_cast<f32x4_t*>(dst + 4) = f32x4_t{s[4], s[5], s[6], s[7]};
          }
          y[((size_t)t * H + h) * kDv + col] = yv;
        };
        Ops a, b;
        fetch(0, a);
        int i = 0;
        for (; i + 1 < mb; i += 2) {
          fetch(i + 1, b);
          token(i, a);
          fetch(min(i + 2, mb - 1), a);
          token(i + 1, b);
        }
        if (i < mb) token(i, a);
      };
      if (states_out)
        chain(BoolTag<true>{});
      else
        chain(BoolTag<false>{});
    }
  }
  if constexpr (kTree) return;  // a draft tree's state is chosen by the commit
  *reinterpret_cast<f32x4_t*>(state + sidx) = f32x4_t{s[0], s[1], s[2], s[3]};
  *reinterpret_cast<f32x4_t*>(state + sidx + 4) = f32x4_t{s[4], s[5], s[6], s[7]};
}

// One token of the gated delta rule with the output norm in the same launch, for a step that keeps
// no per-token state: one workgroup per head, so the head's y never leaves the workgroup. 16-lane
// group cc owns value columns cc and cc + 64 with the recurrence's lane layout (8 key dims per
// lane, gdn_token, the q/k norms formed by group 0 as gdn_kernel's group 0 forms a lone token's),
// so the state and y are bitwise gdn_kernel's. y goes to LDS, and wave 0 forms
// out = rmsnorm(y) * w * silu(z) over the head as gated_rmsnorm_kernel<2> does (lane i holds
// values i and i + 64, the same fma order and wave sum): out is bitwise the two launches'.
constexpr int kHeadThreads = 1024;
constexpr int kHeadGroups = kHeadThreads / kPart;  // 64 lane groups, two value columns each
static_assert(2 * kHeadGroups == kDv, "two value columns per lane group");

__global__ __launch_bounds__(kHeadThreads) void gdn_head_gated_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ bcol, const uint16_t* __restrict__ acol,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias, float* __restrict__ state,
    const uint16_t* __restrict__ z, const uint16_t* __restrict__ norm_w, float eps, uint16_t* __restrict__ out,
    int H, int Hk) {
  __shared__ __attribute__((aligned(16))) uint16_t qk_lds[2][kDk];
  __shared__ __attribute__((aligned(16))) float qkn_lds[2][kDk];  // q * qn, k * kn
  __shared__ uint16_t v_lds[kDv];
  __shared__ float gate_lds[2];  // decay, beta
  __shared__ float y_lds[kDv];
  const int h = blockIdx.x, tid = threadIdx.x;
  const int cc = tid / kPart, p = tid % kPart;
  // The output norm's operands first (wave 0): they depend on nothing.
  uint16_t zv[2] = {0, 0}, wv[2] = {0, 0};
  if (tid < 64) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      zv[j] = z[(size_t)h * kDv + tid + 64 * j];
      wv[j] = norm_w[tid + 64 * j];
    }
  }
  const size_t sidx0 = ((size_t)h * kDv + cc) * kDk + p * 8;   // column cc
  const size_t sidx1 = sidx0 + (size_t)kHeadGroups * kDk;       // column cc + 64
  float s0[8], s1[8];
  {
    const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(state + sidx0);
    const f32x4_t b0 = *reinterpret_cast<const f32x4_t*>(state + sidx0 + 4);
    const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(state + sidx1);
    const f32x4_t b1 = *reinterpret_cast<const f32x4_t*>(state + sidx1 + 4);
    s0[0] = a0.x; s0[1] = a0.y; s0[2] = a0.z; s0[3] = a0.w; s0[4] = b0.x; s0[5] = b0.y; s0[6] = b0.z; s0[7] = b0.w;
    s1[0] = a1.x; s1[1] = a1.y; s1[2] = a1.z; s1[3] = a1.w; s1[4] = b1.x; s1[5] = b1.y; s1[6] = b1.z; s1[7] = b1.w;
  }
  if (tid < 32) {  // q and k: 16 pieces of 16 bytes each
    const int sel = tid >> 4, piece = tid & 15;
    *reinterpret_cast<u32x4_t*>(&qk_lds[sel][piece * 8]) =
        *reinterpret_cast<const u32x4_t*>(qkv + (size_t)sel * Hk * kDk + (size_t)(h / (H / Hk)) * kDk + piece * 8);
  } else if (tid < 32 + kDv) {
    v_lds[tid - 32] = qkv[(size_t)2 * Hk * kDk + (size_t)h * kDv + (tid - 32)];
  } else if (tid == 32 + kDv) {
    gate_lds[0] = expf(-expf(A_log[h]) * softplus(bf16_bits_to_f32(acol[h]) + dt_bias[h]));
  } else if (tid == 33 + kDv) {
    gate_lds[1] = 1.0f / (1.0f + expf(-bf16_bits_to_f32(bcol[h])));
  }
  __syncthreads();
  if (tid < kPart) {  // the token's normalised q and k
    const u32x4_t qw = *reinterpret_cast<const u32x4_t*>(&qk_lds[0][p * 8]);
    const u32x4_t kw = *reinterpret_cast<const u32x4_t*>(&qk_lds[1][p * 8]);
    float q[8], k[8];
    float qq = 0.f, kk = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      q[e] = bf16_bits_to_f32((e & 1) ? (qw[e >> 1] >> 16) : (qw[e >> 1] & 0xffffu));
      k[e] = bf16_bits_to_f32((e & 1) ? (kw[e >> 1] >> 16) : (kw[e >> 1] & 0xffffu));
      qq = fmaf(q[e], q[e], qq);
      kk = fmaf(k[e], k[e], kk);
    }
    const float qn = rsqrtf(sum16(qq) + 1e-6f) * rsqrtf((float)kDk);
    const float kn = rsqrtf(sum16(kk) + 1e-6f);
    f32x4_t* qd = reinterpret_cast<f32x4_t*>(&qkn_lds[0][p * 8]);
    f32x4_t* kd = reinterpret_cast<f32x4_t*>(&qkn_lds[1][p * 8]);
    qd[0] = f32x4_t{q[0] * qn, q[1] * qn, q[2] * qn, q[3] * qn};
    qd[1] = f32x4_t{q[4] * qn, q[5] * qn, q[6] * qn, q[7] * qn};
    kd[0] = f32x4_t{k[0] * kn, k[1] * kn, k[2] * kn, k[3] * kn};
    kd[1] = f32x4_t{k[4] * kn, k[5] * kn, k[6] * kn, k[7] * kn};
  }
  __syncthreads();
  float qh[8], kh[8];
  {
    const f32x4_t* qp = reinterpret_cast<const f32x4_t*>(&qkn_lds[0][p * 8]);
    const f32x4_t* kp = reinterpret_cast<const f32x4_t*>(&qkn_lds[1][p * 8]);
    const f32x4_t q0 = qp[0], q1 = qp[1], k0 = kp[0], k1 = kp[1];
    qh[0] = q0.x; qh[1] = q0.y; qh[2] = q0.z; qh[3] = q0.w; qh[4] = q1.x; qh[5] = q1.y; qh[6] = q1.z; qh[7] = q1.w;
    kh[0] = k0.x; kh[1] = k0.y; kh[2] = k0.z; kh[3] = k0.w; kh[4] = k1.x; kh[5] = k1.y; kh[6] = k1.z; kh[7] = k1.w;
  }
  const float decay = gate_lds[0], beta = gate_lds[1];
  const float y0 = gdn_token(s0, kh, qh, bf16_bits_to_f32(v_lds[cc]), decay, beta);
  const float y1 = gdn_token(s1, kh, qh, bf16_bits_to_f32(v_lds[cc + kHeadGroups]), decay, beta);
  if (p == 0) {
    y_lds[cc] = y0;
    y_lds[cc + kHeadGroups] = y1;
  }
  *reinterpret_cast<f32x4_t*>(state + sidx0) = f32x4_t{s0[0], s0[1], s0[2], s0[3]};
  *reinterpret_cast<f32x4_t*>(state + sidx0 + 4) = f32x4_t{s0[4], s0[5], s0[6], s0[7]};
  *reinterpret_cast<f32x4_t*>(state + sidx1) = f32x4_t{s1[0], s1[1], s1[2], s1[3]};
  *reinterpret_cast<f32x4_t*>(state + sidx1 + 4) = f32x4_t{s1[4], s1[5], s1[6], s1[7]};
  __syncthreads();
  if (tid < 64) {
    const float yv[2] = {y_lds[tid], y_lds[tid + 64]};
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) ss = fmaf(yv[j], yv[j], ss);
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss / (float)kDv + eps);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float gate = silu_gate(bf16_bits_to_f32(zv[j]));
      out[(size_t)h * kDv + tid + 64 * j] = f32_to_bf16_bits(yv[j] * inv * bf16_bits_to_f32(wv[j]) * gate);
    }
  }
}

// Rollback selection over L layers: state[l] = states[l][keep-1], conv_state[l] rows r =
// window[l][keep + r]. keep is read from device memory; keep == fed leaves everything as the
// verify pass left it (the reference's no-op, rollback.py:61-62).
__global__ void gdn_select_kernel(const int32_t* __restrict__ keep_p, int fed, float* __restrict__ state,
                                  const float* __restrict__ states, size_t state_elems, size_t states_stride) {
  const int keep = keep_p[0];
  if (keep < 1 || keep >= fed) return;
  const int l = blockIdx.y;
  const f32x4_t* src = reinterpret_cast<const f32x4_t*>(states + l * states_stride + (size_t)(keep - 1) * state_elems);
  f32x4_t* dst = reinterpret_cast<f32x4_t*>(state + l * state_elems);
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < state_elems / 4; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

__global__ void conv_select_kernel(const int32_t* __restrict__ keep_p, int fed, uint16_t* __restrict__ conv_state,
                                   const uint16_t* __restrict__ window, int rows, int C, size_t window_stride) {
  const int keep = keep_p[0];
  if (keep < 1 || keep >= fed) return;
  const int l = blockIdx.y;
  const size_t n = (size_t)rows * C;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    conv_state[l * n + i] = window[l * window_stride + (size_t)keep * C + i];
}

// Commit of an accepted draft-tree path over L layers. path[0] = count (nodes kept), path[1 ..
// count] = the nodes root .. leaf. state[l] = states[l][leaf]; the conv state becomes the last
// KW-1 inputs of the sequence [old conv state rows; inputs of the path nodes], read from window.
__global__ void gdn_commit_kernel(const int32_t* __restrict__ path, float* __restrict__ state,
                                  const float* __restrict__ states, size_t state_elems, size_t states_stride) {
  const int count = path[0];
  const int l = blockIdx.y;
  const f32x4_t* src =
      reinterpret_cast<const f32x4_t*>(states + l * states_stride + (size_t)path[count] * state_elems);
  f32x4_t* dst = reinterpret_cast<f32x4_t*>(state + l * state_elems);
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < state_elems / 4; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

// The state commit of an accepted draft-tree path by replay, over L layers (grid (H, Dv / kCols,
// L), threads as in gdn_kernel): the state before the step, which a tree pass leaves in place,
// advanced through the path's nodes root .. leaf with the operands the tree pass recorded, by the
// same token update in the same order, so the result is bitwise the leaf's state in that pass.
// path[0] = nodes kept (1 .. kTokBlock), path[1 ..] the nodes.
__global__ __launch_bounds__(kGdnThreads) void gdn_replay_commit_kernel(const int32_t* __restrict__ path,
                                                                        float* __restrict__ state,
                                                                        const float* __restrict__ record,
                                                                        size_t record_stride, int H) {
  const int h = blockIdx.x, l = blockIdx.z, tid = threadIdx.x;
  const int cc = tid / kPart, p = tid % kPart;
  const int col = blockIdx.y * kCols + cc;
  float* st = state + (size_t)l * H * kDv * kDk + ((size_t)h * kDv + col) * kDk + p * 8;
  const float* rec = record + (size_t)l * record_stride;
  const GdnRecord rl(kTokBlock, H);
  const uint16_t* rv = reinterpret_cast<const uint16_t*>(rec + rl.v);
  const int count = min(max(path[0], 1), kTokBlock);
  float s[8];
  {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(st);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(st + 4);
    s[0] = a.x; s[1] = a.y; s[2] = a.z; s[3] = a.w; s[4] = b.x; s[5] = b.y; s[6] = b.z; s[7] = b.w;
  }
  // The path's operands four nodes at a time, all loads of a group issued together.
  constexpr int kGroup = 4;
  for (int j0 = 0; j0 < count; j0 += kGroup) {
    f32x4_t q[kGroup][2], k[kGroup][2];
    float v[kGroup], decay[kGroup], beta[kGroup];
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const int node = min(max(path[1 + min(j0 + j, count - 1)], 0), kTokBlock - 1);
      const float* qk = rec + rl.qk + ((size_t)node * H + h) * 2 * kDk + p * 8;
      q[j][0] = *reinterpret_cast<const f32x4_t*>(qk);
      q[j][1] = *reinterpret_cast<const f32x4_t*>(qk + 4);
      k[j][0] = *reinterpret_cast<const f32x4_t*>(qk + kDk);
      k[j][1] = *reinterpret_cast<const f32x4_t*>(qk + kDk + 4);
      v[j] = bf16_bits_to_f32(rv[(size_t)node * H * kDv + (size_t)h * kDv + col]);
      decay[j] = rec[rl.g + ((size_t)node * H + h) * 2];
      beta[j] = rec[rl.g + ((size_t)node * H + h) * 2 + 1];
    }
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      if (j0 + j >= count) break;
      const float qh[8] = {q[j][0].x, q[j][0].y, q[j][0].z, q[j][0].w, q[j][1].x, q[j][1].y, q[j][1].z, q[j][1].w};
      const float kh[8] = {k[j][0].x, k[j][0].y, k[j][0].z, k[j][0].w, k[j][1].x, k[j][1].y, k[j][1].z, k[j][1].w};
      gdn_token(s, kh, qh, v[j], decay[j], beta[j]);
    }
  }
  *reinterpret_cast<f32x4_t*>(st) = f32x4_t{s[0], s[1], s[2], s[3]};
  *reinterpret_cast<f32x4_t*>(st + 4) = f32x4_t{s[4], s[5], s[6], s[7]};
}

__global__ void conv_commit_kernel(const int32_t* __restrict__ path, uint16_t* __restrict__ conv_state,
                                   const uint16_t* __restrict__ window, int rows, int C, size_t window_stride) {
  const int count = path[0];
  const int l = blockIdx.y;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < (size_t)rows * C; i += (size_t)gridDim.x * blockDim.x) {
    const int r = (int)(i / C), c = (int)(i % C);
    const int q = count + r;  // index in [old rows; path inputs]
    const int wrow = q < rows ? q : rows + path[1 + q - rows];
    conv_state[l * (size_t)rows * C + i] = window[l * window_stride + (size_t)wrow * C + c];
  }
}

}  // namespace

extern "C" int skinny_gdn_conv_silu(const uint16_t* x, int ldx, int M, int C, int KW, uint16_t* conv_state,
                                    const uint16_t* weight, uint16_t* out, int ldo, uint16_t* window,
                                    const int32_t* parent, void* stream) {
  SKINNY_CHECK_ARG(x && conv_state && weight && out, "gdn_conv: null pointer");
  SKINNY_CHECK_ARG(KW == 4, "gdn_conv: kernel width %d unsupported (only 4)", KW);
  SKINNY_CHECK_ARG(M >= 1 && C >= 1 && ldx >= C && ldo >= C, "gdn_conv: bad shape");
  SKINNY_CHECK_ARG(!parent || window, "gdn_conv: a draft tree needs the window buffer");
  SKINNY_CHECK_ARG(!parent || M <= kTokBlock, "gdn_conv: a draft tree holds at most %d tokens (M=%d)", kTokBlock, M);
  hipLaunchKernelGGL(conv_silu_kernel<4>, dim3((C + kConvThreads - 1) / kConvThreads), dim3(kConvThreads), 0,
                     (hipStream_t)stream, x, ldx, M, C, conv_state, weight, out, ldo, window, parent);
  return skinny_check_launch("gdn_conv");
}

extern "C" size_t skinny_gdn_record_words(int H) { return H >= 1 ? GdnRecord(kTokBlock, H).words : 0; }

extern "C" int skinny_gdn_recurrence(const uint16_t* qkv, int ldq, const uint16_t* b, const uint16_t* a, int ldab,
                                     const float* A_log, const float* dt_bias, float* state, float* states_out,
                                     float* y, const int32_t* parent, int M, int H, int Hk, int Dk, int Dv,
                                     float* record, void* stream) {
  SKINNY_CHECK_ARG(qkv && b && a && A_log && dt_bias && state && y, "gdn: null pointer");
  SKINNY_CHECK_ARG(!parent || states_out || record, "gdn: a draft tree needs the per-token states or the record buffer");
  SKINNY_CHECK_ARG(!record || (parent && skinny_aligned(record, 16)),
                   "gdn: the record is a draft tree's, 16-byte aligned");
  SKINNY_CHECK_ARG(Dk == kDk && Dv == kDv, "gdn: head dims %dx%d unsupported (only 128x128)", Dk, Dv);
  SKINNY_CHECK_ARG(M >= 1 && H >= 1 && Hk >= 1 && H % Hk == 0 && ldq >= 2 * Hk * Dk + H * Dv && ldab >= H,
                   "gdn: bad shape M=%d H=%d Hk=%d ldq=%d ldab=%d", M, H, Hk, ldq, ldab);
  SKINNY_CHECK_ARG(!parent || M <= kTokBlock, "gdn: a draft tree holds at most %d tokens (M=%d)", kTokBlock, M);
  SKINNY_CHECK_ARG(skinny_aligned(state, 16) && (!states_out || skinny_aligned(states_out, 16)),
                   "gdn: state buffers must be 16-byte aligned");
  SKINNY_CHECK_ARG(skinny_aligned(qkv, 16) && ldq % 8 == 0, "gdn: qkv rows must be 16-byte aligned");
  const size_t snap_bytes = parent ? (size_t)M * kGdnThreads * 2 * sizeof(f32x4_t) : 0;
  if (snap_bytes > 0) {
    // Dynamic LDS beyond 64 KB (with the static part) must be allowed per kernel; repeating the
    // call is harmless. A 16-node tree's snapshots take 64 KB.
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gdn_kernel<true>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)snap_bytes);
    if (e != hipSuccess) return skinny_set_error(SKINNY_ELAUNCH, "gdn: %zu bytes of snapshots: %s", snap_bytes, hipGetErrorString(e));
  }
  hipLaunchKernelGGL(parent ? gdn_kernel<true> : gdn_kernel<false>, dim3(H, kDv / kCols), dim3(kGdnThreads), snap_bytes,
                     (hipStream_t)stream, qkv, ldq, b, a, ldab, A_log, dt_bias, state, states_out, y, parent, M, H,
                     record, Hk);
  return skinny_check_launch("gdn");
}

extern "C" int skinny_gdn_recurrence_gated_bf16(const uint16_t* qkv, int ldq, const uint16_t* b, const uint16_t* a,
                                                const float* A_log, const float* dt_bias, float* state,
                                                const uint16_t* z, const uint16_t* norm_w, float eps, uint16_t* out,
                                                int H, int Hk, int Dk, int Dv, void* stream) {
  SKINNY_CHECK_ARG(qkv && b && a && A_log && dt_bias && state && z && norm_w && out, "gdn_gated: null pointer");
  SKINNY_CHECK_ARG(Dk == kDk && Dv == kDv, "gdn_gated: head dims %dx%d unsupported (only 128x128)", Dk, Dv);
  SKINNY_CHECK_ARG(H >= 1 && Hk >= 1 && H % Hk == 0 && ldq >= 2 * Hk * Dk + H * Dv,
                   "gdn_gated: bad shape H=%d Hk=%d ldq=%d", H, Hk, ldq);
  SKINNY_CHECK_ARG(skinny_aligned(state, 16), "gdn_gated: the state must be 16-byte aligned");
  SKINNY_CHECK_ARG(skinny_aligned(qkv, 16), "gdn_gated: the qkv row must be 16-byte aligned");
  SKINNY_CHECK_ARG((const void*)out != (const void*)z, "gdn_gated: out must not alias z");
  hipLaunchKernelGGL(gdn_head_gated_kernel, dim3(H), dim3(kHeadThreads), 0, (hipStream_t)stream, qkv, b, a, A_log,
                     dt_bias, state, z, norm_w, eps, out, H, Hk);
  return skinny_check_launch("gdn_gated");
}

extern "C" int skinny_gdn_select(const int32_t* keep, int fed, int layers, float* state, const float* states,
                                 size_t state_elems, size_t states_stride, uint16_t* conv_state, const uint16_t* window,
                                 int conv_rows, int C, size_t window_stride, void* stream) {
  SKINNY_CHECK_ARG(keep && state && states && conv_state && window, "gdn_select: null pointer");
  SKINNY_CHECK_ARG(fed >= 1 && layers >= 1 && state_elems % 4 == 0 && states_stride >= (size_t)fed * state_elems,
                   "gdn_select: bad sizes");
  SKINNY_CHECK_ARG(window_stride >= (size_t)(fed + conv_rows) * C, "gdn_select: window too small");
  SKINNY_CHECK_ARG(skinny_aligned(state, 16) && skinny_aligned(states, 16) && states_stride % 4 == 0,
                   "gdn_select: state buffers must be 16-byte aligned");
  hipLaunchKernelGGL(gdn_select_kernel, dim3(256, layers), dim3(256), 0, (hipStream_t)stream, keep, fed, state, states,
                     state_elems, states_stride);
  int rc = skinny_check_launch("gdn_select");
  if (rc) return rc;
  hipLaunchKernelGGL(conv_select_kernel, dim3(32, layers), dim3(256), 0, (hipStream_t)stream, keep, fed, conv_state,
                     window, conv_rows, C, window_stride);
  return skinny_check_launch("conv_select");
}

extern "C" int skinny_gdn_commit(const int32_t* path, int max_nodes, int layers, float* state, const float* states,
                                 size_t state_elems, size_t states_stride, uint16_t* conv_state, const uint16_t* window,
                                 int conv_rows, int C, size_t window_stride, void* stream) {
  SKINNY_CHECK_ARG(path && state && states && conv_state && window, "gdn_commit: null pointer");
  SKINNY_CHECK_ARG(max_nodes >= 1 && layers >= 1 && state_elems % 4 == 0 &&
                       states_stride >= (size_t)max_nodes * state_elems,
                   "gdn_commit: bad sizes");
  SKINNY_CHECK_ARG(window_stride >= (size_t)(max_nodes + conv_rows) * C, "gdn_commit: window too small");
  SKINNY_CHECK_ARG(skinny_aligned(state, 16) && skinny_aligned(states, 16) && states_stride % 4 == 0,
                   "gdn_commit: state buffers must be 16-byte aligned");
  hipLaunchKernelGGL(gdn_commit_kernel, dim3(256, layers), dim3(256), 0, (hipStream_t)stream, path, state, states,
                     state_elems, states_stride);
  int rc = skinny_check_launch("gdn_commit");
  if (rc) return rc;
  hipLaunchKernelGGL(conv_commit_kernel, dim3(32, layers), dim3(256), 0, (hipStream_t)stream, path, conv_state, window,
                     conv_rows, C, window_stride);
  return skinny_check_launch("conv_commit");
}

extern "C" int skinny_gdn_commit_replay(const int32_t* path, int layers, int H, float* state, const float* record,
                                        size_t record_stride, uint16_t* conv_state, const uint16_t* window,
                                        int conv_rows, int C, size_t window_stride, void* stream) {
  SKINNY_CHECK_ARG(path && state && record && conv_state && window, "gdn_commit_replay: null pointer");
  SKINNY_CHECK_ARG(layers >= 1 && H >= 1 && record_stride >= GdnRecord(kTokBlock, H).words && record_stride % 4 == 0,
                   "gdn_commit_replay: bad sizes");
  SKINNY_CHECK_ARG(window_stride >= (size_t)(kTokBlock + conv_rows) * C, "gdn_commit_replay: window too small");
  SKINNY_CHECK_ARG(skinny_aligned(state, 16) && skinny_aligned(record, 16),
                   "gdn_commit_replay: state and record must be 16-byte aligned");
  hipLaunchKernelGGL(gdn_replay_commit_kernel, dim3(H, kDv / kCols, layers), dim3(kGdnThreads), 0, (hipStream_t)stream,
                     path, state, record, record_stride, H);
  int rc = skinny_check_launch("gdn_commit_replay");
  if (rc) return rc;
  hipLaunchKernelGGL(conv_commit_kernel, dim3(32, layers), dim3(256), 0, (hipStream_t)stream, path, conv_state, window,
                     conv_rows, C, window_stride);
  return skinny_check_launch("conv_commit");
}
