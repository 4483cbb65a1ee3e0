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
 * K, N and the tile (never on M), so outputs are bitwise identical for any M.
 * rf/sk/ns select the tile: 16-row tiles per wave (1 or 2), waves per
 * workgroup splitting the K/128 group pairs (1, 2, 4, 8 or 16, at most K/128;
 * uneven splits allowed) and ns, the ring of group pairs each wave keeps in
 * flight (2..5; 16-wave workgroups allow 4 at rf=1 and 3 at rf=2); pass 0 for
 * all three to use the table.
 */
int skinny_qmm_w4g64_bf16(const uint16_t* x, int M, int K, int ldx,
                          const uint32_t* w_frag, int N, uint16_t* y, int ldy,
                          int rf, int sk, int ns, void* stream);

/* Tile the table picks for (K, N); writes rf/sk/ns. Keyed by (K, N) only. */
int skinny_qmm_pick_tile(int K, int N, int* rf, int* sk, int* ns);

/* ---------------------------------------------------------------------------
 * Streaming-read ceiling (harness). Reads `bytes` (multiple of 16, 16-byte aligned)
 * with `grid` workgroups of 256 threads and writes one value per workgroup to out[grid]
 * so the reads cannot be elided. Counterpart of bench/hw_roofline.py:3-11.
 */
int skinny_stream_read(const void* buf, size_t bytes, float* out, int grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SKINNY_HIP_H */
