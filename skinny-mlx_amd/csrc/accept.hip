// Greedy acceptance of the verify step, on the device.
//
// Reference behaviour: skinny_mlx/spec.py:137-147 — pred = argmax over each verify row
// (mx.argmax: the first maximal index), n = the longest prefix with draft[i] == pred[i],
// emitted tokens draft[:n] + [pred[n]], cache rolled back to keep = n + 1 of fed = K + 1.
#include "common.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kArgmaxLoads = 20;  // 16-byte pieces per thread in one round trip: V <= 163840

// (value, index) with first-index ties: larger value wins, equal values keep the lower index.
__device__ __forceinline__ void better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// Element e of a 16-byte piece of bf16 values.
__device__ __forceinline__ float piece_at(const u32x4_t& w, int e) {
  return bf16_bits_to_f32((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
}

// One workgroup per row; bf16 logits with row stride ld. A 16-byte aligned row is read in
// 16-byte pieces (8 logits), several loads in flight per thread; the rest one value at a time.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const uint16_t* __restrict__ logits, int V, int ld,
                                                          int32_t* __restrict__ pred) {
  const uint16_t* row = logits + (size_t)blockIdx.x * ld;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const int nv = skinny_aligned(row, 16) ? V >> 3 : 0;
  const u32x4_t* r4 = reinterpret_cast<const u32x4_t*>(row);
  // A thread visits its logits in increasing index order, so a strictly larger value is the only
  // update its first-index rule needs (NaN never compares larger); threads then combine with the
  // full (value, index) rule.
  auto take = [&](float v, int ix) {
    if (v > bv) {
      bv = v;
      bi = ix;
    }
  };
  if (nv <= kArgmaxLoads * kThreads) {
    // The whole row in one round trip: every piece's load issued before the first is compared (a
    // thread past the row's end reloads its last piece, and skips it).
    u32x4_t w[kArgmaxLoads];
#pragma unroll
    for (int j = 0; j < kArgmaxLoads; ++j) w[j] = r4[min((int)threadIdx.x + j * kThreads, max(nv - 1, 0))];
#pragma unroll
    for (int j = 0; j < kArgmaxLoads; ++j) {
      const int i = threadIdx.x + j * kThreads;
      if (i < nv)
#pragma unroll
        for (int e = 0; e < 8; ++e) take(piece_at(w[j], e), 8 * i + e);
    }
  } else {
#pragma unroll 4
    for (int i = threadIdx.x; i < nv; i += kThreads) {
      const u32x4_t w = r4[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) take(piece_at(w, e), 8 * i + e);
    }
  }
  for (int i = 8 * nv + threadIdx.x; i < V; i += kThreads) take(bf16_bits_to_f32(row[i]), i);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) better(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
  __shared__ float sv[kThreads / 64];
  __shared__ int si[kThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w) better(bv, bi, sv[w], si[w]);
    pred[blockIdx.x] = bi == 0x7fffffff ? 0 : bi;
  }
}

// out[0] = n (accepted drafts), out[1] = bonus token pred[n], out[2] = keep = n + 1.
__global__ void accept_kernel(const int32_t* __restrict__ pred, const int32_t* __restrict__ draft, int k,
                              int32_t* __restrict__ out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int n = 0;
  while (n < k && draft[n] == pred[n]) ++n;
  out[0] = n;
  out[1] = pred[n];
  out[2] = n + 1;
}

// The end of a verify step of a decode loop that stays on the device, after accept_kernel or
// tree_accept_kernel (res = [n, bonus, keep, ...], 1 <= keep <= fed): the verify pass advanced
// the cache length by fed, and it moves back to the kept tokens (*pos += keep - fed, the KV
// trim); the tokens the step emits -- the predictions at the kept rows, which for the accepted
// drafts equal the drafts, then the bonus: pred[j] for a chain, pred[sel[j]] along a tree's path
// -- are appended to tokens at *count (slots at or past cap are not written) and *count grows by
// keep; *next = the bonus (res[1]), the first token of the next verify pass. One wave: every lane
// reads *count before lane 0 writes it (one load, then one store instruction).
__global__ __launch_bounds__(64) void spec_commit_kernel(const int32_t* __restrict__ res, int fed,
                                                         int32_t* __restrict__ pos, const int32_t* __restrict__ pred,
                                                         const int32_t* __restrict__ sel, int32_t* __restrict__ tokens,
                                                         int32_t* __restrict__ count, int cap,
                                                         int32_t* __restrict__ next) {
  const int keep = min(max(res[2], 1), fed);
  const int c = count[0];
  const int j = threadIdx.x;
  if (j < keep && c + j < cap) tokens[c + j] = pred[sel ? min(max(sel[j], 0), fed - 1) : j];
  __syncthreads();
  if (j == 0) {
    count[0] = c + keep;
    pos[0] += keep - fed;
    next[0] = res[1];
  }
}

// dst = row keep - 1 of rows (H bf16 values, row stride ld; keep = res[2], 1 <= keep <= fed), and
// *pos += keep - fed: a drafter's state after a pass over all fed rows of which keep count.
__global__ __launch_bounds__(256) void spec_select_row_kernel(const int32_t* __restrict__ res, int fed,
                                                              int32_t* __restrict__ pos,
                                                              const uint16_t* __restrict__ rows, int ld, int H,
                                                              uint16_t* __restrict__ dst) {
  const int keep = min(max(res[2], 1), fed);
  const uint16_t* src = rows + (size_t)(keep - 1) * ld;
  for (int i = threadIdx.x; i < H; i += blockDim.x) dst[i] = src[i];
  if (threadIdx.x == 0) pos[0] += keep - fed;
}

// Draft-tree acceptance: from the root (node 0), repeatedly step to the first child (in node
// order) whose token equals the prediction at the current node; stop when none does. Writes
// out[0] = n (accepted drafts = path length - 1), out[1] = bonus = pred at the last node,
// out[2] = count = n + 1, out[3 .. 3 + n] = the path's nodes. A chain (parent i - 1) is exactly
// the linear acceptance.
__global__ void tree_accept_kernel(const int32_t* __restrict__ pred, const int32_t* __restrict__ tokens,
                                   const int32_t* __restrict__ parent, int M, int32_t* __restrict__ out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int cur = 0, n = 0;
  out[3] = 0;
  for (;;) {
    int next = -1;
    for (int c = cur + 1; c < M; ++c)
      if (parent[c] == cur && tokens[c] == pred[cur]) {
        next = c;
        break;
      }
    if (next < 0) break;
    ++n;
    out[3 + n] = next;
    cur = next;
  }
  out[0] = n;
  out[1] = pred[cur];
  out[2] = n + 1;
}

// Top-k of each row of bf16 logits: indices of the k largest values, in decreasing value order,
// equal values ordered by index. One workgroup per row: every thread keeps a sorted list of the
// best kTopK of its strided elements, lists are merged pairwise through LDS in a fixed tree, and
// the first k of the row's best kTopK are written (the first k of a top-kTopK list are the top k).
constexpr int kTopK = 8;
constexpr int kTopKLoads = 8;  // 16-byte pieces per thread in one round trip: V <= 65536

__device__ __forceinline__ bool ranks_before(float v, int i, float v2, int i2) { return v > v2 || (v == v2 && i < i2); }

__global__ __launch_bounds__(kThreads) void topk_kernel(const uint16_t* __restrict__ logits, int V, int ld, int k,
                                                        int32_t* __restrict__ idx_out) {
  __shared__ float sv[kThreads][kTopK];
  __shared__ int si[kThreads][kTopK];
  const uint16_t* row = logits + (size_t)blockIdx.x * ld;
  float bv[kTopK];
  int bi[kTopK];
#pragma unroll
  for (int j = 0; j < kTopK; ++j) {
    bv[j] = -INFINITY;
    bi[j] = 0x7fffffff;
  }
  // A thread offers its logits in increasing index order, so a new value ranks before the last
  // kept one only when it is strictly larger (an equal one has the higher index), or equal to the
  // empty slot's -inf (whose index is larger than any).
  auto offer = [&](float v, int ix) {
    if (!(v > bv[kTopK - 1]) && !(v == bv[kTopK - 1] && bi[kTopK - 1] == 0x7fffffff)) return;
#pragma unroll
    for (int j = 0; j < kTopK; ++j) {  // insertion: the displaced entry moves one place down
      if (v > bv[j] || (v == bv[j] && ix < bi[j])) {
        const float tv = bv[j];
        const int ti = bi[j];
        bv[j] = v;
        bi[j] = ix;
        v = tv;
        ix = ti;
      }
    }
  };
  const int nv = skinny_aligned(row, 16) ? V >> 3 : 0;  // 16-byte pieces, as in argmax_kernel
  const u32x4_t* r4 = reinterpret_cast<const u32x4_t*>(row);
  if (nv <= kTopKLoads * kThreads) {  // one round trip, as in argmax_kernel
    u32x4_t w[kTopKLoads];
#pragma unroll
    for (int j = 0; j < kTopKLoads; ++j) w[j] = r4[min((int)threadIdx.x + j * kThreads, max(nv - 1, 0))];
#pragma unroll
    for (int j = 0; j < kTopKLoads; ++j) {
      const int i = threadIdx.x + j * kThreads;
      if (i < nv)
#pragma unroll
        for (int e = 0; e < 8; ++e) offer(piece_at(w[j], e), 8 * i + e);
    }
  } else {
#pragma unroll 2
    for (int i = threadIdx.x; i < nv; i += kThreads) {
      const u32x4_t w = r4[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) offer(piece_at(w, e), 8 * i + e);
    }
  }
  for (int i = 8 * nv + threadIdx.x; i < V; i += kThreads) offer(bf16_bits_to_f32(row[i]), i);
#pragma unroll
  for (int j = 0; j < kTopK; ++j) {
    sv[threadIdx.x][j] = bv[j];
    si[threadIdx.x][j] = bi[j];
  }
  __syncthreads();
  for (int stride = kThreads / 2; stride > 0; stride >>= 1) {
    if ((int)threadIdx.x < stride) {
      const int o = threadIdx.x + stride;
      float mv[kTopK];
      int mi[kTopK];
      int a = 0, b = 0;
#pragma unroll
      for (int j = 0; j < kTopK; ++j) {
        const bool take_a = ranks_before(sv[threadIdx.x][a], si[threadIdx.x][a], sv[o][b], si[o][b]);
        mv[j] = take_a ? sv[threadIdx.x][a] : sv[o][b];
        mi[j] = take_a ? si[threadIdx.x][a] : si[o][b];
        a += take_a;
        b += !take_a;
      }
#pragma unroll
      for (int j = 0; j < kTopK; ++j) {
        sv[threadIdx.x][j] = mv[j];
        si[threadIdx.x][j] = mi[j];
      }
    }
    __syncthreads();
  }
  if ((int)threadIdx.x < k) {
    const int ix = si[0][threadIdx.x];
    idx_out[(size_t)blockIdx.x * k + threadIdx.x] = ix == 0x7fffffff ? 0 : ix;
  }
}

// Compaction of an accepted draft-tree path in the attention caches of L layers: the path's
// node at depth d moves from slot p0 + path[1 + d] to slot p0 + d (path[0] = count), where
// p0 = pos[0] - pos_back is the tree's first slot. Each thread owns one head dimension and walks
// the depths in order, so a slot is always read before a later depth overwrites it.
__global__ void kv_commit_kernel(const int32_t* __restrict__ path, const int32_t* __restrict__ pos, int pos_back,
                                 uint16_t* kc, uint16_t* vt, int Hkv, int maxlen, int D, size_t layer_stride) {
  const int lh = blockIdx.x, d = threadIdx.x;
  if (d >= D) return;
  const int l = lh / Hkv, h = lh % Hkv;
  const int count = path[0];
  const int p0 = pos[0] - pos_back;
  uint16_t* kh = kc + l * layer_stride + (size_t)h * maxlen * D;
  uint16_t* vh = vt + l * layer_stride + (size_t)h * D * maxlen;
  for (int dep = 1; dep < count; ++dep) {
    const int src = p0 + path[1 + dep], dst = p0 + dep;
    if (src == dst) continue;
    kh[(size_t)dst * D + d] = kh[(size_t)src * D + d];
    vh[(size_t)d * maxlen + dst] = vh[(size_t)d * maxlen + src];
  }
}

}  // namespace

extern "C" int skinny_argmax_rows_bf16(const uint16_t* logits, int rows, int V, int ld, int32_t* pred, void* stream) {
  SKINNY_CHECK_ARG(logits && pred, "argmax: null pointer");
  SKINNY_CHECK_ARG(rows >= 1 && V >= 1 && ld >= V, "argmax: bad shape rows=%d V=%d ld=%d", rows, V, ld);
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, logits, V, ld, pred);
  return skinny_check_launch("argmax");
}

extern "C" int skinny_accept(const int32_t* pred, const int32_t* draft, int k, int32_t* out, void* stream) {
  SKINNY_CHECK_ARG(pred && out && (k == 0 || draft), "accept: null pointer");
  SKINNY_CHECK_ARG(k >= 0, "accept: k=%d must be >= 0", k);
  hipLaunchKernelGGL(accept_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, pred, draft, k, out);
  return skinny_check_launch("accept");
}

extern "C" int skinny_spec_commit(const int32_t* res, int fed, int32_t* pos, const int32_t* pred, const int32_t* sel,
                                  int32_t* tokens, int32_t* count, int cap, int32_t* next, void* stream) {
  SKINNY_CHECK_ARG(res && pos && pred && tokens && count && next, "spec_commit: null pointer");
  SKINNY_CHECK_ARG(fed >= 1 && fed <= 64, "spec_commit: fed=%d must be in [1, 64]", fed);
  SKINNY_CHECK_ARG(cap >= 0, "spec_commit: cap=%d must be >= 0", cap);
  hipLaunchKernelGGL(spec_commit_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, res, fed, pos, pred, sel, tokens,
                     count, cap, next);
  return skinny_check_launch("spec_commit");
}

extern "C" int skinny_spec_select_row(const int32_t* res, int fed, int32_t* pos, const uint16_t* rows, int ld, int H,
                                      uint16_t* dst, void* stream) {
  SKINNY_CHECK_ARG(res && pos && rows && dst, "spec_select_row: null pointer");
  SKINNY_CHECK_ARG(fed >= 1 && fed <= 64, "spec_select_row: fed=%d must be in [1, 64]", fed);
  SKINNY_CHECK_ARG(H >= 1 && ld >= H, "spec_select_row: bad shape H=%d ld=%d", H, ld);
  hipLaunchKernelGGL(spec_select_row_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, res, fed, pos, rows, ld, H,
                     dst);
  return skinny_check_launch("spec_select_row");
}

extern "C" int skinny_tree_accept(const int32_t* pred, const int32_t* tokens, const int32_t* parent, int M, int32_t* out,
                                  void* stream) {
  SKINNY_CHECK_ARG(pred && tokens && parent && out, "tree_accept: null pointer");
  SKINNY_CHECK_ARG(M >= 1 && M <= 64, "tree_accept: M=%d must be in [1, 64]", M);
  hipLaunchKernelGGL(tree_accept_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, pred, tokens, parent, M, out);
  return skinny_check_launch("tree_accept");
}

extern "C" int skinny_topk_rows_bf16(const uint16_t* logits, int rows, int V, int ld, int k, int32_t* idx,
                                     void* stream) {
  SKINNY_CHECK_ARG(logits && idx, "topk: null pointer");
  SKINNY_CHECK_ARG(rows >= 1 && V >= 1 && ld >= V && k >= 1 && k <= kTopK && k <= V, "topk: bad shape rows=%d V=%d k=%d",
                   rows, V, k);
  hipLaunchKernelGGL(topk_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, logits, V, ld, k, idx);
  return skinny_check_launch("topk");
}

extern "C" int skinny_kv_commit(const int32_t* path, const int32_t* pos, int pos_back, uint16_t* k_cache,
                                uint16_t* vt_cache, int layers, int Hkv, int maxlen, int D, size_t layer_stride,
                                void* stream) {
  SKINNY_CHECK_ARG(path && pos && k_cache && vt_cache, "kv_commit: null pointer");
  SKINNY_CHECK_ARG(pos_back >= 0, "kv_commit: pos_back=%d must be >= 0", pos_back);
  SKINNY_CHECK_ARG(layers >= 1 && Hkv >= 1 && D >= 1 && D <= 1024 && maxlen >= 1 &&
                       layer_stride >= (size_t)Hkv * maxlen * D,
                   "kv_commit: bad shape");
  hipLaunchKernelGGL(kv_commit_kernel, dim3(layers * Hkv), dim3((D + 63) / 64 * 64), 0, (hipStream_t)stream, path, pos,
                     pos_back, k_cache, vt_cache, Hkv, maxlen, D, layer_stride);
  return skinny_check_launch("kv_commit");
}
