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

#define SKINNY_ABI_VERSION 1

/* Error codes. */
#define SKINNY_OK 0
#define SKINNY_EINVAL -1   /* bad shape, pointer, alignment or argument */
#define SKINNY_ELAUNCH -2  /* HIP launch / runtime error */
#define SKINNY_ESPACE -3   /* caller workspace too small */

int skinny_abi_version(void);
const char* skinny_last_error(void);

/* ---------------------------------------------------------------------------
 * W4 g64 weight relayout (load time).
 * Replaces repack_for_skinny (skinny_mlx/qmm.py:96-115): the same bytes in a
 * different order. Fragment order is [N/16 tiles][K/64 groups][64 lanes][2 u32];
 * lane l of tile t, group g, half h holds row 16t + l%16, columns
 * 64g + 32h + 8(l/16) + 0..7, element 2i at bits 4i and element 2i+1 at bits
 * 16+4i. Requires N % 16 == 0, K % 64 == 0, 4-byte aligned buffers.
 */
int skinny_w4g64_relayout(const uint32_t* w_mlx, uint32_t* w_frag, int N, int K, void* stream);
/* Inverse of skinny_w4g64_relayout (fragment order back to MLX packs). */
int skinny_w4g64_unrelayout(const uint32_t* w_frag, uint32_t* w_mlx, int N, int K, void* stream);

/* ---------------------------------------------------------------------------
 * W4A16 g64 skinny quantized matmul: y[M,N] = x[M,K] . dequant(w)[N,K]^T.
 * Replaces the Metal kernel skinny_qmm_4bit and its host wrapper skinny_qmm
 * (skinny_mlx/qmm.py:21-93, 132-152) and, for M = 1..5, mx.quantized_matmul
 * (skinny_mlx/patch.py:30-35).
 *   x      [M,K] bf16, row stride ldx elements (ldx >= K, ldx % 8 == 0), 16-byte aligned
 *   w_frag fragment-order nibbles from skinny_w4g64_relayout
 *   scales, biases [N, K/64] bf16 (MLX layout, untouched)
 *   y      [M,N] bf16, row stride ldy elements (ldy >= N)
 *   1 <= M <= 16, K % 128 == 0, N % 16 == 0.
 * Accumulation is fp32; the result for a token row depends only on that row,
 * K, N and the tile (never on M), so outputs are bitwise identical for any M.
 * rf/sk/ks select the tile (row tiles per wave, waves per workgroup splitting
 * K, workgroups splitting K); pass 0 for all three to use the built-in table.
 * ks > 1 needs `workspace` (fp32, zero-initialised once by the caller; the
 * counters it holds are reset by the kernel itself) of at least
 * skinny_qmm_workspace_bytes(...) bytes; otherwise workspace may be NULL.
 */
int skinny_qmm_w4g64_bf16(const uint16_t* x, int M, int K, int ldx,
                          const uint32_t* w_frag, const uint16_t* scales, const uint16_t* biases,
                          int N, uint16_t* y, int ldy,
                          int rf, int sk, int ks,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Tile the table picks for (K, N); writes rf/sk/ks. Keyed by (K, N) only. */
int skinny_qmm_pick_tile(int K, int N, int* rf, int* sk, int* ks);
/* Workspace bytes needed for (N, tile). */
size_t skinny_qmm_workspace_bytes(int N, int rf, int sk, int ks);

#ifdef __cplusplus
}
#endif

#endif /* SKINNY_HIP_H */
