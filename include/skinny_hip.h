/*
 * skinny_hip.h — C ABI of libskinny_hip.so, the MI355X (gfx950) kernels of the
 * flat-cost speculative-verify path.
 *
 * Conventions shared by every entry point:
 *   - All functions are extern "C", return 0 on success and a negative code on
 *     failure; skinny_last_error() then holds a message (thread-local).
 *   - Every pointer argument named as a device buffer is device memory the caller
 *     allocated (PyTorch tensors in the Python host layer). The library never
 *     allocates or frees device memory and keeps no reference to caller buffers.
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default
 *     stream). Work is enqueued asynchronously; no entry point synchronises,
 *     allocates or copies to the host, so every one can be captured in a HIP
 *     graph.
 *   - bf16 values travel as uint16_t bit patterns.
 *   - "W4 g64" is MLX's affine 4-bit format: w[n,k] = q[n,k]*s[n,k/64] + b[n,k/64],
 *     q packed eight per little-endian uint32 with element i at bits 4i.
 */
#ifndef SKINNY_HIP_H
#define SKINNY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SKINNY_ABI_VERSION 19

/* Error codes. */
#define SKINNY_OK 0
#define SKINNY_EINVAL -1   /* bad shape, pointer, alignment or argument */
#define SKINNY_ELAUNCH -2  /* HIP launch / runtime error */

int skinny_abi_version(void);
const char* skinny_last_error(void);

/* ---------------------------------------------------------------------------
 * W4 g64 weight packing (load time).
 * Replaces repack_for_skinny (skinny_mlx/qmm.py:96-115): the same nibbles in a
 * different order, with the scales and biases moved next to them. The packed
 * buffer holds N/16 x K/128 blocks of 288 u32 (1152 bytes), block (t, p) at word
 * (t*K/128 + p)*288:
 *   words [0, 256):   lane l, word 2j+h at 4l + 2j + h holds row 16t + l%16,
 *                     columns 64(2p+j) + 32h + 8(l/16) + e, e = 0..7, with e < 4
 *                     in the low nibble of byte e and e+4 in its high nibble;
 *   words [256, 288): row r at 256 + 2r: scales of groups 2p, 2p+1 (low, high
 *                     16 bits), then biases of the same two groups.
 * Packed size: N*(K/8 + K/64) u32. Requires N % 16 == 0, K % 128 == 0, w_mlx and
 * scales/biases ([N, K/64] bf16, MLX layout) naturally aligned, w_frag 16-byte
 * aligned and distinct from w_mlx.
 */
int skinny_w4g64_pack(const uint32_t* w_mlx, const uint16_t* scales, const uint16_t* biases,
                      uint32_t* w_frag, int N, int K, void* stream);
/* Inverse of skinny_w4g64_pack: back to MLX packs, scales and biases. */
int skinny_w4g64_unpack(const uint32_t* w_frag, uint32_t* w_mlx, uint16_t* scales, uint16_t* biases,
                        int N, int K, void* stream);

/* The nibbles alone, for the reference's one-argument relayout: replaces
 * `repack_for_skinny(w)` (skinny_mlx/qmm.py:96-115), "same bytes, different order",
 * [N, K/8] u32 in, [N, K/8] u32 out. Block (t, p) of 256 u32 at word (t*K/128 + p)*256
 * holds words [0, 256) of skinny_w4g64_pack's block. Both buffers 16-byte aligned and
 * distinct; N % 16 == 0, K % 128 == 0. */
int skinny_w4g64_relayout(const uint32_t* w_mlx, uint32_t* w_frag, int N, int K, void* stream);
/* Inverse of skinny_w4g64_relayout. */
int skinny_w4g64_unrelayout(const uint32_t* w_frag, uint32_t* w_mlx, int N, int K, void* stream);
/* skinny_w4g64_pack's buffer from a skinny_w4g64_relayout result plus MLX-layout scales and
 * biases ([N, K/64] bf16): what `skinny_qmm(x, w, scales, biases)` (skinny_mlx/qmm.py:132)
 * reads, completed once per (relayout, scales, biases). */
int skinny_w4g64_attach(const uint32_t* w_frag, const uint16_t* scales, const uint16_t* biases,
                        uint32_t* packed, int N, int K, void* stream);

/* ---------------------------------------------------------------------------
 * W4A16 g64 skinny quantized matmul: y[M,N] = x[M,K] . dequant(w)[N,K]^T.
 * Replaces the Metal kernel skinny_qmm_4bit and its host wrapper skinny_qmm
 * (skinny_mlx/qmm.py:21-93, 132-152) and, for M = 1..5, mx.quantized_matmul
 * (skinny_mlx/patch.py:30-35).
 *   x      [M,K] bf16, row stride ldx elements (ldx >= K, ldx % 8 == 0), 16-byte aligned
 *   w_frag packed weights, scales and biases from skinny_w4g64_pack
 *   y      [M,N] bf16, row stride ldy elements (ldy >= N)
 *   1 <= M <= 16, K % 128 == 0, N % 16 == 0.
 * Accumulation is fp32; the result for a token row depends only on that row,
 * K, N and the tile (never on M), and every sum runs in a fixed order, so
 * outputs are bitwise identical for any M and any run.
 *   tile   NULL = the table's tile for (K, N) (skinny_qmm_pick_tile).
 */
#define SKINNY_QMM_WAVE_X 1 /* each wave loads its own X fragments; waves split K */
#define SKINNY_QMM_SLAB_X 2 /* X staged once per workgroup in LDS; waves split rows */
typedef struct skinny_qmm_tile {
  int kind;  /* SKINNY_QMM_WAVE_X or SKINNY_QMM_SLAB_X */
  int rf;    /* 16-row tiles per wave sharing each X fragment: 1, 2 or 4 (N/16 must
                divide by it) */
  int waves; /* waves per workgroup. WAVE_X: they split the K/128 group pairs (1, 2,
                4, 8, 16; at most K/128; uneven splits allowed). SLAB_X: they own
                different row tiles and each walks all of K (1..8); K <= 3072 (the
                slab holds 4 KB of X per group pair) */
  int ns;    /* group pairs each wave keeps in flight. WAVE_X: 2..5 (rf=4: 2..3; 16-wave
                workgroups: at most 4 at rf=1, 3 at rf=2, none at rf=4). SLAB_X: 2, 3,
                4, 6 (rf <= 2), 8 (rf = 1) */
} skinny_qmm_tile;

int skinny_qmm_w4g64_bf16(const uint16_t* x, int M, int K, int ldx,
                          const uint32_t* w_frag, int N, uint16_t* y, int ldy,
                          const skinny_qmm_tile* tile, void* stream);

/* Tile the table picks for (K, N). Keyed by (K, N) only. */
int skinny_qmm_pick_tile(int K, int N, skinny_qmm_tile* tile);

/* skinny_qmm_w4g64_bf16 with `splits` (2..4) workgroups sharing each row tile group's K, for
 * shapes whose N gives too few row tiles to fill the GPU (the o_proj/down shapes, N = 2560): the
 * first splits-1 publish fp32 sums with device-coherent stores into `workspace`, the last adds
 * them in split order, rounds and stores y. The workspace (skinny_qmm_splitk_workspace_bytes(N,
 * splits) bytes, 16-byte aligned: a 16-byte header, then the slices) must have every 32-bit word
 * 0xFFFFFFFF ("not yet written") before its first use — fill it once after allocating it; every
 * call leaves it so. Calls that share a workspace must be ordered (one stream): give each stream
 * that may run such calls at the same time as another its own workspace. A last split that waits
 * in vain (a bounded poll) writes NaN and sets the header's first word; from then on every call
 * with that workspace writes NaN rows until the caller replaces (or refills) it. A token's row
 * still depends only on that row, K, N, the tile and `splits`. tile NULL with the table's choice:
 * skinny_qmm_splitk_pick. */
int skinny_qmm_w4g64_splitk_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N,
                                 uint16_t* y, int ldy, float* workspace, size_t workspace_bytes, int splits,
                                 const skinny_qmm_tile* tile, void* stream);
size_t skinny_qmm_splitk_workspace_bytes(int N, int splits);
/* The measured split and tile for (K, N); splits = 1 (and skinny_qmm_pick_tile's tile) where the
 * unsplit kernel is faster. */
int skinny_qmm_splitk_pick(int K, int N, int* splits, skinny_qmm_tile* tile);

/* Fused same-input gate|up projection (patch.py:23-27 fuses gate_proj and up_proj along N)
 * with the SwiGLU activation of the MLP folded into its epilogue.
 *   w_frag  skinny_w4g64_pack of the 2F x K weight whose row tiles alternate gate and up:
 *           packed tile 2j = gate rows 16j..16j+15, tile 2j+1 = up rows 16j..16j+15.
 *   swiglu  0: y [M, 2F] = [x.gate^T | x.up^T] in the unfused column order;
 *           1: y [M, F] = silu(gate) * up, from the bf16-rounded projections — bitwise what
 *              skinny_silu_mul_bf16 makes of the swiglu = 0 output.
 *   tile    NULL = skinny_qmm_glu_pick_tile(K, F); rf must be 2 (one wave owns a gate and
 *           an up tile). `waves` is the number of K groups whose sums are added in group
 *           order: the library may run a tile's groups on fewer waves for some token counts
 *           (the 4-group tile over K = 2560 runs as one wave from M = 2 on), with the same
 *           products, so a token's row never depends on M.
 */
int skinny_qmm_w4g64_glu_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int F,
                              uint16_t* y, int ldy, int swiglu, const skinny_qmm_tile* tile, void* stream);
/* Tile of the gate|up layout: the table's tile for (K, 2F) with rf = 2. */
int skinny_qmm_glu_pick_tile(int K, int F, skinny_qmm_tile* tile);

/* The MLP sublayer of the decoder in one launch (the reference plan's "~1 dispatch per sublayer",
 * docs/roofline-and-plan.md:93; the gate/up fusion of patch.py:23-27 and the down projection after
 * it): part = the split-K fp32 slices [3][M][N] of skinny_qmm_w4g64_partial_f32(silu(x gate^T) *
 * (x up^T), w_down), bitwise the gate|up launch (skinny_qmm_w4g64_glu_bf16 with swiglu = 1) followed
 * by that partial launch. Workgroups of the gate|up tile publish their SwiGLU columns into `act`
 * ([M][F] bf16, row stride F) and count them in `sync`; the down tiles, dispatched after them, issue
 * their weight loads at once and wait (a bounded poll: NaN, never a hang, if a count never arrives)
 * only for the 128-column groups they read. `sync`: skinny_mlp_fused_sync_bytes(F) bytes, zero
 * before the first call; every call leaves it zero, so calls sharing it must be ordered (one
 * stream). For M = 2..16 and the (K, F, N) whose tiles have the fused instance: the gate|up tile's
 * one-wave form and the (3 splits, rf 2, 4 waves, ring 3) down tile (skinny_mlp_fused_supported;
 * the 36-layer decoders' 2560 -> 2 x 9728 -> 2560). The wait assumes the device to itself, as
 * skinny_qkv_attention_fused_bf16's does: a down tile that gives up writes NaN and no error is
 * reported. */
int skinny_mlp_fused_partial_f32(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_gate_up, int F,
                                 const uint32_t* w_down, int N, uint16_t* act, float* part, uint32_t* sync,
                                 size_t sync_bytes, void* stream);
int skinny_mlp_fused_supported(int M, int K, int F, int N);
size_t skinny_mlp_fused_sync_bytes(int F);

/* Split-K form for projections whose output feeds a residual RMSNorm (o_proj, the MLP down
 * projection, the Gated-DeltaNet out_proj; each is the residual of the next norm in the decoder
 * the reference patches, spec.py:24-29): `splits` workgroups share each row tile's K, each
 * writing fp32 sums over its share of the group pairs, unrounded, to part[s][t][n] (slice s at
 * s * M * ldp floats, row stride ldp >= N). skinny_rmsnorm_partials_bf16 adds the slices. The tile
 * must be wave-X with waves <= (K/128) / splits; splits <= 4. skinny_qmm_partial_pick gives the
 * measured split and tile for (K, N). */
int skinny_qmm_w4g64_partial_f32(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N, float* part,
                                 int ldp, int splits, const skinny_qmm_tile* tile, void* stream);
/* skinny_qmm_w4g64_partial_f32 of the Gated-DeltaNet output norm, formed inside the launch: X =
 * bf16(rmsnorm(y) * norm_w * silu(z)) per head of 128 values (K = heads x 128, so a group pair is
 * one head), from y fp32 [M, K] (row stride ldy) and z bf16 [M, K] (row stride ldz), with the
 * (K, N) split-K tile and splits of skinny_qmm_partial_pick. X is bitwise skinny_gated_rmsnorm's
 * output (each lane forms the sum of squares of its head in that kernel's order), so the slices
 * are bitwise that kernel followed by skinny_qmm_w4g64_partial_f32: one launch fewer per
 * Gated-DeltaNet layer. SKINNY_EINVAL where no gated-norm-in kernel exists for the tile
 * (skinny_qmm_gated_partial_supported). No counterpart in the reference, whose layer runs the
 * norm (mlx_lm) and the projection as separate ops. */
int skinny_qmm_w4g64_gated_partial_f32(const float* y, int ldy, const uint16_t* z, int ldz, const uint16_t* norm_w,
                                       float eps, int M, int K, const uint32_t* w_frag, int N, float* part, int ldp,
                                       void* stream);
int skinny_qmm_gated_partial_supported(int K, int N);
int skinny_qmm_partial_pick(int K, int N, int* splits, skinny_qmm_tile* tile);

/* Norm-in forms (no counterpart in the reference, whose decoder runs each RMSNorm as its own op
 * before the projections, spec.py:24-29): the projection of X = rmsnorm(v) * weight with
 * v = bf16(h + bf16(sum of `splits` fp32 slices in order)) (v = h when splits = 0), formed inside
 * the matmul launch. X, and v stored to h_out, are bitwise what skinny_rmsnorm_partials_bf16 (or
 * skinny_rmsnorm_bf16 without slices) gives, and the product bitwise skinny_qmm_w4g64_bf16 /
 * skinny_qmm_w4g64_glu_bf16 (swiglu) / skinny_qmm_w4g64_conv_bf16 of that X with the same tile.
 * Every workgroup forms all of X from the rows (for few tokens that costs less than the separate
 * norm launch it replaces). h [M, K] and the slices [splits, M, K] are contiguous; h_out must not
 * be h. M <= 4; skinny_qmm_normin_supported says whether a tile (NULL: the shape's default) has a
 * norm-in kernel and the rows fit its LDS (1 when the call would run). */
typedef struct skinny_norm_in {
  const uint16_t* h;       /* [M, K] bf16: the residual stream before the add */
  const float* parts;      /* [splits, M, K] fp32: slices of the residual projection, or NULL */
  int splits;              /* 0..4 (0 exactly when parts is NULL) */
  const uint16_t* weight;  /* [K] bf16 norm weight */
  float eps;
  uint16_t* h_out;         /* [M, K] bf16: receives v (the residual stream after the add), or NULL */
} skinny_norm_in;
#define SKINNY_NORMIN_PLAIN 0
#define SKINNY_NORMIN_SWIGLU 1
#define SKINNY_NORMIN_CONV 2
int skinny_qmm_normin_supported(int kind, int M, int K, int N, int splits, const skinny_qmm_tile* tile);
int skinny_qmm_w4g64_normin_bf16(const skinny_norm_in* ni, int M, int K, const uint32_t* w_frag, int N, uint16_t* y,
                                 int ldy, const skinny_qmm_tile* tile, void* stream);
int skinny_qmm_w4g64_glu_normin_bf16(const skinny_norm_in* ni, int M, int K, const uint32_t* w_frag, int F,
                                     uint16_t* y, int ldy, const skinny_qmm_tile* tile, void* stream);
int skinny_qmm_w4g64_conv_normin_bf16(const skinny_norm_in* ni, int M, int K, const uint32_t* w_frag, int N,
                                      uint16_t* y, int ldy, int C, uint16_t* conv_state, const uint16_t* conv_w,
                                      int KW, uint16_t* window, const int32_t* parent, const skinny_qmm_tile* tile,
                                      void* stream);
/* The fused Gated-DeltaNet input projection (q|k|v|z|b|a, the GDN member of patch.py:23-27's
 * FUSE_GROUPS) with the mixer's short causal conv + SiLU (the conv whose input rollback.py:44-52
 * records) applied to its first C columns in the same launch: y[:, :C] is bitwise what
 * skinny_gdn_conv_silu makes of skinny_qmm_w4g64_bf16's output (conv_state advanced, window
 * recorded, draft-tree parents followed the same way), y[:, C:] the plain output. M <= 16, KW = 4,
 * C a multiple of 16. tile == NULL picks a wave-X tile. */
int skinny_qmm_w4g64_conv_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N, uint16_t* y,
                               int ldy, int C, uint16_t* conv_state, const uint16_t* conv_w, int KW, uint16_t* window,
                               const int32_t* parent, const skinny_qmm_tile* tile, void* stream);
/* ---------------------------------------------------------------------------
 * Decoder glue of the verify forward (the mlx_lm model the reference patches and runs at
 * skinny_mlx/spec.py:24-29). bf16 in/out, fp32 arithmetic; every op is per row, so results
 * do not depend on how many tokens share a launch.
 */
/* out = rmsnorm(x (+ residual)) * weight; with sum_out, also stores x + residual (bf16),
 * which may alias x (in-place residual add). rows x H. */
int skinny_rmsnorm_bf16(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, float eps,
                        uint16_t* out, uint16_t* sum_out, int rows, int H, void* stream);
/* skinny_rmsnorm_bf16 with the residual given as `splits` fp32 slices of a split-K matmul (slice
 * s at s * split_stride floats, row stride ldp): residual = bf16(slice 0 + slice 1 + ...), in
 * split order. */
int skinny_rmsnorm_partials_bf16(const uint16_t* x, const float* parts, int splits, size_t split_stride, int ldp,
                                 const uint16_t* weight, float eps, uint16_t* out, uint16_t* sum_out, int rows, int H,
                                 void* stream);
/* The MTP head's input (mtp.py:51-67: fc([rms_e(embed(tok)); rms_h(h)])) up to the fc projection,
 * in one launch: out[t, 0:H] = rmsnorm(table[ids[t]]) * w_e, out[t, H:2H] = rmsnorm(hidden[t]) * w_h
 * (hidden rows of stride ldh), bit for bit what skinny_embed_bf16 and two skinny_rmsnorm_bf16 calls
 * give, concatenated. ids out of [0, V) are clamped as skinny_embed_bf16 clamps them. */
int skinny_mtp_input_bf16(const int32_t* ids, int tokens, const uint16_t* table, int V, const uint16_t* hidden,
                          int ldh, const uint16_t* w_e, const uint16_t* w_h, float eps, uint16_t* out, int H,
                          void* stream);
/* Gated-DeltaNet output norm: out[t,h,:] = rmsnorm(y[t,h,:]) * weight * silu(z[t,h,:]);
 * y fp32 [tokens, heads, D], z bf16 rows of stride ldz; D a multiple of 64, at most 1024. */
int skinny_gated_rmsnorm(const float* y, const uint16_t* z, int ldz, const uint16_t* weight, float eps,
                         uint16_t* out, int tokens, int heads, int D, void* stream);
/* SwiGLU: act[t, i] = silu(gate_up[t, i]) * gate_up[t, F + i] (the fused gate|up
 * projection of patch.py:23-27), rows of stride ld. */
int skinny_silu_mul_bf16(const uint16_t* gate_up, int ld, uint16_t* act, int tokens, int F, void* stream);
/* Embedding gather: out[t] = table[ids[t]] (bf16 [V, H] table). */
int skinny_embed_bf16(const int32_t* ids, int tokens, const uint16_t* table, int V, int H, uint16_t* out,
                      void* stream);
/* W4 g64 dequantisation to fp32 [N, K] (q*s + b in fp32): the unpatched linear path, the
 * semantics of mx.quantized_matmul that patch.py:35 keeps for M outside SKINNY_RANGE. */
int skinny_w4g64_dequant(const uint32_t* w_mlx, const uint16_t* scales, const uint16_t* biases,
                         float* out, int N, int K, void* stream);

/* Attention layers. Cache per layer: K [Hkv][maxlen][D], V transposed [Hkv][D][maxlen],
 * bf16; *pos0 (device) = tokens cached before this step; the step's M tokens go to cache
 * slots pos0 .. pos0+M-1 (mlx_lm KVCache append, trimmed at rollback.py:71-73).
 *
 * Draft trees (`tree`, NULL = the causal chain): an int32 descriptor of 1 + 2M entries.
 * tree[0] = b: the tree's keys occupy slots [pos0 - b, pos0 - b + 32); tree[1 + t] = the bit
 * mask over those 32 slots of the keys token t sees there (its ancestors and itself);
 * tree[1 + M + t] = token t's RoPE position relative to pos0 (its depth). Keys before the tree
 * are visible to every token, keys after it to none. A chain — b = 0, masks 2^(t+1) - 1,
 * positions t — computes exactly what NULL computes.
 *
 * skinny_qk_rope_store: from fused q|k|v rows (stride ldq), per-head RMSNorm of q and k
 * (weights may be NULL to skip), rotate-half RoPE with base theta, q to q_out [M, Hq, D], k and
 * v into the caches at slot pos0 + t. D must be 128; with a tree, M <= 32. */
int skinny_qk_rope_store(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D,
                         const uint16_t* q_norm, const uint16_t* k_norm, float eps, const int32_t* pos0,
                         float theta, const int32_t* tree, uint16_t* q_out, uint16_t* k_cache,
                         uint16_t* vt_cache, int maxlen, void* stream);
/* GQA attention of q [M, Hq, D] over the cache (keys 0 .. pos0+M-1; causal: query t sees keys
 * <= pos0+t; or as `tree` says) -> out [M, Hq, D] bf16. (Hq/Hkv)*M <= 64, D = 128,
 * maxlen % 128 == 0; needs an fp32 workspace of skinny_attn_workspace_bytes(Hkv, maxlen) bytes
 * (no initialisation). */
size_t skinny_attn_workspace_bytes(int Hkv, int maxlen);
int skinny_attention_bf16(const uint16_t* q, int M, int Hq, int Hkv, int D, const uint16_t* k_cache,
                          const uint16_t* vt_cache, int maxlen, const int32_t* pos0, float scale,
                          const int32_t* tree, float* workspace, size_t workspace_bytes, uint16_t* out,
                          void* stream);
/* skinny_qk_rope_store followed by skinny_attention_bf16 in one fewer launch (the "norm + QKV +
 * RoPE" fusion the reference plans, docs/roofline-and-plan.md:93): from the step's raw q|k|v rows
 * (stride ldq, a multiple of 8), the query rows are normalised and rotated inside the attention
 * kernel, and the new key/value rows are written to the caches there. RoPE factors come from
 * `rope_table` ([rope_positions][64] (cos, sin) fp32, skinny_rope_table), rope_positions >=
 * maxlen. M <= 16; otherwise as the two calls it replaces (the K cache holds the same bits). */
int skinny_attention_fused_bf16(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D, const uint16_t* q_norm,
                                const uint16_t* k_norm, float eps, const float* rope_table, int rope_positions,
                                const int32_t* pos0, const int32_t* tree, uint16_t* k_cache, uint16_t* vt_cache,
                                int maxlen, float scale, float* workspace, size_t workspace_bytes, uint16_t* out,
                                void* stream);
/* The fused q|k|v projection of an attention layer (patch.py:23-27's same-input group: y = x .
 * w_frag^T, N = (Hq + 2 Hkv) D) and skinny_attention_fused_bf16 over its rows, in one launch plus
 * the chunk merge. The projection's workgroups publish the q|k|v rows into `handoff` ([>= M]
 * rows of N bf16, row stride ld_handoff, a multiple of 8); the attention's chunk workgroups load
 * the device position and their KV chunk while the projection streams its weights, then wait for
 * the rows they need. Every 16-bit word of rows 0..M-1 (N columns) of `handoff` must hold 0xFFFF
 * before the call (fill it once after allocating it); the merge puts them back, so calls that
 * share a buffer must be ordered (one stream). The projection takes the (K, N) table's tile
 * (skinny_qmm_pick_tile), so its rows are bitwise skinny_qmm_w4g64_bf16's, and out, the caches and
 * the partials are those of skinny_qmm_w4g64_bf16 followed by skinny_attention_fused_bf16.
 * SKINNY_EINVAL where no fused kernel exists for that tile or the launch would not fit on the GPU
 * at once (skinny_qkv_attention_supported); the caller then takes the two calls. The fit is
 * counted on an idle GPU and the wait is bounded: with kernels of other streams running at the same
 * time, a chunk workgroup can give up before its rows arrive and write NaN, and the call reports no
 * error, so this form needs the device to itself (callers that overlap streams take the two calls).
 * No counterpart in the reference, where the projection and the attention are separate MLX ops. */
int skinny_qkv_attention_fused_bf16(const uint16_t* x, int M, int K, int ldx, const uint32_t* w_frag, int N,
                                    uint16_t* handoff, int ld_handoff, int Hq, int Hkv, int D,
                                    const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                    const float* rope_table, int rope_positions, const int32_t* pos0,
                                    const int32_t* tree, uint16_t* k_cache, uint16_t* vt_cache, int maxlen,
                                    float scale, float* workspace, size_t workspace_bytes, uint16_t* out,
                                    void* stream);
/* 1 when skinny_qkv_attention_fused_bf16 runs for (K, N, Hkv, maxlen) on the current device, 0
 * when it does not, a negative code when the device cannot be queried. */
int skinny_qkv_attention_supported(int K, int N, int Hkv, int maxlen);
/* skinny_attention_fused_bf16 without the workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The chunk partials live in a file-scope device array of this
 * library (8.1 MiB per GPU, held until the process ends), so Hkv * maxlen / 128 <= 256 (e.g. 8 kv
 * heads over 4096 cached positions); larger shapes return SKINNY_EINVAL. The array's device address
 * is looked up on the first call on each device (hipGetSymbolAddress): make that first call
 * outside a graph capture. The stream must belong to the current device. Every call on one GPU
 * shares its array, so calls that overlap on one GPU (different streams without ordering) race;
 * calls on one stream are ordered. Nothing in the array needs clearing between calls. */
int skinny_attention_fused_noalloc_bf16(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D,
                                        const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                        const float* rope_table, int rope_positions, const int32_t* pos0,
                                        const int32_t* tree, uint16_t* k_cache, uint16_t* vt_cache, int maxlen,
                                        float scale, uint16_t* out, void* stream);
/* table[pos][i] = (cos, sin)(pos * theta^(-2i/128)), i < 64, pos < positions: the factors
 * skinny_qk_rope_store computes inline. */
int skinny_rope_table(float theta, int positions, float* table, void* stream);
/* table[pos][i] = (cos, sin)(pos * theta^(-2i/R)), i < R/2, pos < positions: the factors of a RoPE
 * over the first R = rotary_dim dims of each head (R even, <= 256), by the same expressions; R =
 * 128 gives skinny_rope_table's table. */
int skinny_rope_table_dim(float theta, int rotary_dim, int positions, float* table, void* stream);

/* Full attention for the head layouts the 128-dim kernels above do not take: the attention layers
 * of mlx_lm's Qwen3.5 decoder that the reference loads (spec.py:175) and runs at spec.py:24-29 —
 * q/k RMSNorm, rotate-half RoPE over the first rotary_dim dims of each head, causal GQA
 * attention (or a draft tree, as skinny_attention_bf16), and optionally the attention output
 * gated by sigmoid(gate) (transformers qwen3_5 Attention: q_proj holds per head the query rows,
 * then the gate rows).
 *   qkv        M rows (stride ldq) holding query head h at h * q_stride, key head j at k_offset +
 *              j * D, value head j at v_offset + j * D, and with gate_offset >= 0 the gate of
 *              query head h at gate_offset + h * q_stride (gate_offset < 0: no gate). Qwen3.5:
 *              q_stride = 2D, gate_offset = D, k_offset = 2 Hq D, v_offset = (2 Hq + Hkv) D.
 *   D          64, 128 or 256; rotary_dim even, <= D; rope_table from skinny_rope_table_dim with
 *              the same rotary_dim, rope_positions >= maxlen.
 *   out        [M, Hq * D] bf16: attention(q, K, V) per head, times bf16(sigmoid(gate)) when
 *              gated (both factors rounded to bf16 first).
 * The new keys and values go into the caches (layout as skinny_attention_bf16), the normalised
 * queries and chunk partials into `workspace` (skinny_attn_general_workspace_bytes(Hq, Hkv, D,
 * maxlen) bytes, 256-byte aligned). M <= 16 and (Hq / Hkv) * M <= 64. Three launches. */
int skinny_attention_general_bf16(const uint16_t* qkv, int ldq, int M, int Hq, int Hkv, int D, int q_stride,
                                  int k_offset, int v_offset, int gate_offset, const uint16_t* q_norm,
                                  const uint16_t* k_norm, float eps, int rotary_dim, const float* rope_table,
                                  int rope_positions, const int32_t* pos0, const int32_t* tree,
                                  uint16_t* k_cache, uint16_t* vt_cache, int maxlen, float scale, void* workspace,
                                  size_t workspace_bytes, uint16_t* out, void* stream);
size_t skinny_attn_general_workspace_bytes(int Hq, int Hkv, int D, int maxlen);
/* Accepted draft-tree path into the attention caches of `layers` layers (K and V^T of layer l
 * at l * layer_stride elements): with p0 = *pos - pos_back the tree's first slot, the node at
 * depth d moves from slot p0 + path[1 + d] to slot p0 + d, d = 1 .. path[0] - 1 (path[0] =
 * nodes kept, path[1] = 0, the root). The tree counterpart of the KV trim at rollback.py:71-73;
 * the reference verifies chains only (draft trees are its stated next step, README.md:84). */
int skinny_kv_commit(const int32_t* path, const int32_t* pos, int pos_back, uint16_t* k_cache,
                     uint16_t* vt_cache, int layers, int Hkv, int maxlen, int D, size_t layer_stride,
                     void* stream);

/* Gated-DeltaNet layers (mlx_lm gated_delta_update hooked at rollback.py:16, 39-42; conv
 * input recorded at rollback.py:44-52). State per layer: [H][Dv][Dk] fp32.
 * `parent` (NULL = the chain): for a draft tree of M <= 16 tokens, parent[t] < t is token t's
 * parent, -1 for the root; every token then continues from its parent's state and conv inputs,
 * and neither the state nor the conv state is advanced (skinny_gdn_commit picks the accepted
 * path's).
 * skinny_gdn_conv_silu: causal depthwise conv (width KW = 4) over [conv_state; x] then SiLU;
 * conv_state [KW-1, C] is advanced in place (chain); with `window` non-NULL the M+KW-1 input
 * rows are kept ([M+KW-1, C]) for rollback (required with a tree). */
int skinny_gdn_conv_silu(const uint16_t* x, int ldx, int M, int C, int KW, uint16_t* conv_state,
                         const uint16_t* weight, uint16_t* out, int ldo, uint16_t* window,
                         const int32_t* parent, void* stream);
/* Recurrence over M tokens: q,k l2-normalised (q also scaled by Dk^-1/2), decay
 * g = exp(-exp(A_log) * softplus(a + dt_bias)), beta = sigmoid(b);
 * S <- g S; S <- S + beta (v - S k) k^T; y = S q. state is advanced in place (chain); with
 * states_out non-NULL every per-token state S_1..S_M is also stored ([M][H][Dv][Dk]). A draft
 * tree needs states_out or `record` (NULL for a chain): skinny_gdn_record_words(H) fp32 words,
 * 16-byte aligned, into which the tree pass writes each node's update operands (normalised q and
 * k, decay, beta, v) for skinny_gdn_commit_replay. qkv rows (stride ldq): q [Hk][Dk] | k [Hk][Dk]
 * | v [H][Dv]; H value heads (the state's heads, and of a, b, A_log, dt_bias) read the Hk key
 * heads in groups: value head h reads key head h / (H / Hk) (Qwen3.5's 16 key heads over 32 value
 * heads: q and k repeat_interleave'd, transformers qwen3_5 GatedDeltaNet). b, a: per-head columns
 * with row stride ldab. y: fp32 [M, H, Dv]. Dk = Dv = 128. */
int skinny_gdn_recurrence(const uint16_t* qkv, int ldq, const uint16_t* b, const uint16_t* a, int ldab,
                          const float* A_log, const float* dt_bias, float* state, float* states_out,
                          float* y, const int32_t* parent, int M, int H, int Hk, int Dk, int Dv, float* record,
                          void* stream);
size_t skinny_gdn_record_words(int H);
/* One token of skinny_gdn_recurrence (a chain step that keeps no per-token state) with the GDN
 * output norm of skinny_gated_rmsnorm in the same launch: out [H*Dv] bf16 =
 * rmsnorm(y) * norm_w * silu(z) per head, bitwise the two calls' output, and state advanced
 * bitwise as skinny_gdn_recurrence advances it; the fp32 y is not written. qkv, b, a: the token's
 * row (q | k | v; per-head columns), z: its H*Dv gate values. Replaces, for one token, the
 * pair above (mlx_lm's gated delta step as skinny_mlx/rollback.py:16, 39-42 hooks it, then the
 * mixer's output norm). */
int skinny_gdn_recurrence_gated_bf16(const uint16_t* qkv, int ldq, const uint16_t* b, const uint16_t* a,
                                     const float* A_log, const float* dt_bias, float* state,
                                     const uint16_t* z, const uint16_t* norm_w, float eps, uint16_t* out,
                                     int H, int Hk, int Dk, int Dv, void* stream);
/* Replay-free rollback over `layers` GDN layers (rollback.py:58-73): with keep = *keep
 * (device), if 1 <= keep < fed: state[l] = states[l][keep-1] and conv_state[l] rows r =
 * window[l][keep + r]; otherwise nothing changes (keep == fed is the reference's no-op).
 * Layer l's buffers start at l*state_elems, l*states_stride, l*conv_rows*C and
 * l*window_stride elements. */
int skinny_gdn_select(const int32_t* keep, int fed, int layers, float* state, const float* states,
                      size_t state_elems, size_t states_stride, uint16_t* conv_state, const uint16_t* window,
                      int conv_rows, int C, size_t window_stride, void* stream);
/* The same for an accepted draft-tree path (path[0] = nodes kept, path[1 ..] = root .. leaf,
 * at most max_nodes): state[l] = states[l][leaf]; the conv state becomes the last conv_rows
 * inputs of [old conv state rows; inputs of the path's nodes]. Always applied. The tree
 * counterpart of rollback.py:58-73 (no reference counterpart for trees, README.md:84). */
int skinny_gdn_commit(const int32_t* path, int max_nodes, int layers, float* state, const float* states,
                      size_t state_elems, size_t states_stride, uint16_t* conv_state, const uint16_t* window,
                      int conv_rows, int C, size_t window_stride, void* stream);
/* skinny_gdn_commit from a tree pass's record instead of its node states: every layer's state
 * (layer l at l*H*Dv*Dk; the tree pass leaves it as it was before the step) is advanced through
 * the path's nodes root .. leaf with the recorded operands, by the tree pass's own token update
 * in the same order, so it becomes bitwise the leaf's state; layer l's record at l*record_stride
 * words. The conv state as skinny_gdn_commit. The tree pass then writes 330 KB of operands per
 * layer instead of 1 MB of state per node. No reference counterpart (trees: README.md:84). */
int skinny_gdn_commit_replay(const int32_t* path, int layers, int H, float* state, const float* record,
                             size_t record_stride, uint16_t* conv_state, const uint16_t* window, int conv_rows,
                             int C, size_t window_stride, void* stream);

/* Greedy acceptance (spec.py:137-147): pred[r] = first index of the row maximum of bf16
 * logits (rows x V, stride ld); then out[0] = n = longest prefix with draft[i] == pred[i]
 * (i < k), out[1] = pred[n] (bonus token), out[2] = n + 1 (tokens kept). */
int skinny_argmax_rows_bf16(const uint16_t* logits, int rows, int V, int ld, int32_t* pred, void* stream);
int skinny_accept(const int32_t* pred, const int32_t* draft, int k, int32_t* out, void* stream);
/* The end of a verify step of a decode loop kept on the device (no host round trip per step),
 * after skinny_accept or skinny_tree_accept (res = its out, 1 <= keep = res[2] <= fed):
 * *pos += keep - fed (the cache length back to the kept tokens: the KV trim of
 * rollback.py:71-73 on the device length); the tokens the step emits (spec.py:139-141),
 * pred[0 .. keep) -- or pred[sel[j]], j < keep, along a tree's path (sel = res + 3) --
 * appended to tokens at *count, slots >= cap not written; *count += keep; *next = res[1] (the
 * bonus, first token of the next pass). The reference's loop does this on the host after its
 * one mx.eval (spec.py:138-150). */
int skinny_spec_commit(const int32_t* res, int fed, int32_t* pos, const int32_t* pred, const int32_t* sel,
                       int32_t* tokens, int32_t* count, int cap, int32_t* next, void* stream);
/* dst = rows[keep - 1] (H bf16 values, row stride ld; keep = res[2], 1 <= keep <= fed) and
 * *pos += keep - fed: the MTP drafter's update (spec.py:89-95) after a head pass over all fed
 * rows, on the device: its last accepted hidden state and its cache trimmed to the kept rows. */
int skinny_spec_select_row(const int32_t* res, int fed, int32_t* pos, const uint16_t* rows, int ld, int H,
                           uint16_t* dst, void* stream);
/* Greedy acceptance over a draft tree of M nodes (node 0 = the root, parent[i] < i): from the
 * root, step to the first child (node order) whose token equals the prediction at the current
 * node, until none does. out[0] = n accepted drafts, out[1] = bonus (pred at the last node),
 * out[2] = n + 1, out[3 .. 3+n] = the path's nodes (out + 2 is the path form the commits read).
 * No counterpart in the reference, which verifies chains only (its stated next step,
 * README.md:84). */
int skinny_tree_accept(const int32_t* pred, const int32_t* tokens, const int32_t* parent, int M, int32_t* out,
                       void* stream);
/* Indices of the k <= 8 largest values of each bf16 row (decreasing; ties by index): the MTP
 * drafter's top-k for draft trees. Extends the drafter's argmax (spec.py:85) to k candidates;
 * no reference counterpart (draft trees are its stated next step, README.md:84). */
int skinny_topk_rows_bf16(const uint16_t* logits, int rows, int V, int ld, int k, int32_t* idx, void* stream);

/* Sampling at temperature T > 0 and speculative rejection sampling: the reference's stated next
 * step after greedy acceptance (docs/flatspec-design.md:19, item F6; README.md:84), the standard
 * speculative sampling (Leviathan et al. 2023). Random numbers: Philox4x32-10 keyed by `seed`,
 * counter (n, rng_stream) with n = *counter + offset (+ row), *counter read from device memory
 * so captured steps draw fresh numbers on every replay; a uniform is the top 24 bits of the
 * first output word times 2^-24. Sampling is a deterministic inverse CDF over the row.
 *
 * skinny_random_uniform: out[i] = the uniform of n = *counter + offset + i.
 * skinny_row_stats_bf16: stats[r] = (max, sum over the row of exp((x - max) / T)).
 * skinny_sample_rows_bf16: out[r] = a sample of softmax(row r / T), uniform n = *counter +
 *   offset + r. */
int skinny_random_uniform(uint64_t seed, const int64_t* counter, int64_t offset, int n, int rng_stream, float* out,
                          void* stream);
int skinny_row_stats_bf16(const uint16_t* logits, int rows, int V, int ld, float inv_temp, float* stats,
                          void* stream);
int skinny_sample_rows_bf16(const uint16_t* logits, int rows, int V, int ld, float inv_temp, uint64_t seed,
                            const int64_t* counter, int64_t offset, int rng_stream, int32_t* out, void* stream);
/* One speculative step at temperature T: target logits rows 0..K (stride ldt) with their
 * row stats, draft logits rows 0..K-1 over the draft vocabulary [0, Vd) with theirs (draft NULL:
 * the drafts are point masses, e.g. prompt lookup), the K drafts. Draft i is accepted when
 * u_i * q_i(x_i) < p_i(x_i), u_i the uniform of n = *counter + 2i; at the first rejection the
 * emitted token samples max(0, p_i - q_i), else the bonus samples p_K, with n = *counter + 2n + 1.
 * out = [n accepted, emitted token, n + 1], the form of skinny_accept. */
int skinny_spec_accept_sampled(const uint16_t* target, int ldt, const float* stats_t, const uint16_t* draft, int ldd,
                               const float* stats_d, int Vd, const int32_t* drafts, int K, int V, float inv_temp,
                               uint64_t seed, const int64_t* counter, int32_t* out, void* stream);

/* ---------------------------------------------------------------------------
 * Streaming-read ceiling (harness). Reads `bytes` (multiple of 16, 16-byte aligned)
 * with `grid` workgroups of 256 threads and writes one value per workgroup to out[grid]
 * so the reads cannot be elided. Counterpart of bench/hw_roofline.py:3-11.
 */
int skinny_stream_read(const void* buf, size_t bytes, float* out, int grid, void* stream);
/* The same read with each of the `grid` workgroups taking one contiguous chunk of the buffer and
 * `loads` (4, 8 or 16) 16-byte loads in flight per thread: the best of both forms over grids is
 * the ceiling the qmm launches are compared with. */
int skinny_stream_read_chunked(const void* buf, size_t bytes, float* out, int grid, int loads, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SKINNY_HIP_H */
