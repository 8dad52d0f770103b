/* hydraserve_amd: MI355X (gfx950) quantized weight-only linear layers.
 *
 * C ABI of libhydraserve_amd.so.  Plain pointers and sizes only; every device
 * pointer is caller-owned memory on the current HIP device, every call is
 * enqueued on `stream` with no host synchronisation and no allocation, so the
 * calls are safe under HIP graph capture.
 *
 * Return value: 0 on success, otherwise an HS_E* code (see hs_error_string).
 *
 * Data layouts (exactly the reference's tensors, no repacking):
 *   INT4 ("compressed-tensors" asymmetric, group 128):
 *     packed     int32 [N, ceil(K/8)]   nibble i of word j = W[n, 8j+i]
 *     scale      bf16/f16/f32 [N, ceil(K/128)]
 *     zero_point int32 [ceil(N/8), ceil(K/128)]  nibble j of word [r,g] = zp[8r+j, g]
 *   FP8 (E4M3FN, 128x128 blocks):
 *     data       uint8 [N, K]
 *     scale_inv  bf16/f16/f32 [ceil(N/128), ceil(K/128)]
 *   Activations X: bf16 [M, K]; output Y: bf16 [M, N]; strides in elements
 *   (INT4 packed: int32 words; FP8 data: bytes).
 */
#ifndef HYDRASERVE_AMD_H
#define HYDRASERVE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* error codes */
#define HS_OK 0
#define HS_EINVAL 1        /* bad shape, stride, pointer or enum */
#define HS_EWORKSPACE 2    /* workspace missing or smaller than hs_gemm_workspace_bytes() */
#define HS_EUNSUPPORTED 3  /* valid request this library does not implement (e.g. group != 128) */
#define HS_ESCRATCH 4      /* hs_int4_gemm_noalloc: the problem needs more workspace than its fixed scratch */
#define HS_EHIP 1000       /* HS_EHIP + hipError_t from a HIP runtime call */

/* scale / output dtype codes */
#define HS_DT_BF16 0
#define HS_DT_F16 1
#define HS_DT_F32 2

/* weight kinds for hs_gemm_workspace_bytes */
#define HS_KIND_INT4 0
#define HS_KIND_FP8 1

/* ABI version of this header (bumped on any signature change). */
int hs_abi_version(void);

/* Static text for an error code. */
const char* hs_error_string(int code);

/* Bytes of device workspace hs_int4_gemm / hs_fp8_gemm need for this problem
 * on the current device (0 if none).  The workspace holds a fixed 1 MiB
 * block of per-tile arrival counters followed by fp32 partial tiles of the K
 * split.  Problems with more than 2^18 output tiles return HS_EUNSUPPORTED.  It must be zero-filled once
 * when allocated; every call leaves it zero-filled again, so it can be reused
 * by later calls on the same stream.  Calls that overlap in time (different
 * streams) must use different workspaces. */
int64_t hs_gemm_workspace_bytes(int kind, int M, int N, int K);

/* Y[M,N] = X[M,K] . dequant(W)^T, fp32 accumulation, bf16 output.
 * Replaces the GPU branch of awq_linear (hydraserve/kernels/awq.py:25-75,
 * Triton kernel awq.py:82-142).  group must be 128 (awq.py:30-31). */
int hs_int4_gemm(const void* x, int64_t ldx,
                 const int32_t* packed, int64_t ld_packed,
                 const void* scale, int64_t ld_scale, int scale_dtype,
                 const int32_t* zero_point, int64_t ld_zero,
                 void* y, int64_t ldy,
                 int M, int N, int K, int group,
                 void* workspace, int64_t workspace_bytes,
                 void* stream);

/* hs_int4_gemm without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture that may not call
 * hipMalloc, tight serving loops, harnesses that forbid allocation).  No
 * counterpart in the reference.  The split-K workspace is a fixed device
 * array inside the library, one per GPU, of 40 MiB (held from library load
 * until the process ends): problems whose
 * plan needs more return HS_ESCRATCH (at the BASELINE shapes: every M up to
 * 64; prefill M >= 129 does not fit).  The call allocates nothing.  All calls on one GPU
 * share that GPU's array, so calls that overlap in time on one GPU (two
 * streams, two threads) race; serialise them.  Results are those of
 * hs_int4_gemm. */
int hs_int4_gemm_noalloc(const void* x, int64_t ldx,
                         const int32_t* packed, int64_t ld_packed,
                         const void* scale, int64_t ld_scale, int scale_dtype,
                         const int32_t* zero_point, int64_t ld_zero,
                         void* y, int64_t ldy,
                         int M, int N, int K, int group,
                         void* stream);

/* The MLP's gate_up projection with SiLU-and-mul fused into the GEMM's store:
 * out[M, N/2] = silu(gate) * up, gate and up being the bf16 outputs of
 * hs_int4_gemm on W.  Replaces the gate_up _linear call, the chunk and the
 * silu_and_mul launch of hydraserve/model/runtime.py:1202-1210
 * (silu_and_mul: hydraserve/kernels/activation.py:4-25, kernel :66-76).
 * W's rows interleave the gate and up halves in 16-row blocks (gate rows
 * 16j..16j+15, then up rows 16j..16j+15: the load-time layout
 * hydraserve_amd.kernels.mlp.interleave_gate_up builds).  N (both halves) a
 * multiple of 32, ldy >= N/2; workspace as for hs_int4_gemm.  Returns
 * HS_EUNSUPPORTED when K or the strides do not suit the kernels (K a
 * multiple of 128, 16-byte aligned rows; at 1..16 rows K at least 1024); the caller then runs hs_int4_gemm and the activation
 * separately. */
int hs_int4_gemm_silu_mul(const void* x, int64_t ldx,
                          const int32_t* packed, int64_t ld_packed,
                          const void* scale, int64_t ld_scale, int scale_dtype,
                          const int32_t* zero_point, int64_t ld_zero,
                          void* y, int64_t ldy,
                          int M, int N, int K, int group,
                          void* workspace, int64_t workspace_bytes,
                          void* stream);

/* hs_int4_gemm_silu_mul with a load-time tiled copy of the interleaved
 * gate_up weight (layout as for hs_int4_gemm_tiled; same fused branch,
 * hydraserve/model/runtime.py:1202-1210).  Up to 64 rows the tiled decode
 * kernel's store carries the activation (each 16-row gate tile and the up
 * tile after it are settled in one workgroup); from 129 rows the 256x256
 * prefill kernel reads the tiles; 17..128 rows and shapes the tiled kernels
 * do not take run as hs_int4_gemm_silu_mul on the row-major weight.  Results
 * are those of hs_int4_gemm_silu_mul to the same bars. */
int hs_int4_gemm_silu_mul_tiled(const void* x, int64_t ldx,
                                const int32_t* packed, int64_t ld_packed, const int32_t* tiles,
                                const void* scale, int64_t ld_scale, int scale_dtype,
                                const int32_t* zero_point, int64_t ld_zero,
                                void* y, int64_t ldy,
                                int M, int N, int K, int group,
                                void* workspace, int64_t workspace_bytes,
                                void* stream);

/* Y[M,N] = X[M,K] . (decode(W) * scale_inv[n/128, k/128])^T, fp32 accumulation,
 * bf16 output.  Replaces the GPU branch of fp8_linear
 * (hydraserve/kernels/fp8.py:24-97, Triton kernel fp8.py:104-168). */
int hs_fp8_gemm(const void* x, int64_t ldx,
                const uint8_t* data, int64_t ld_data,
                const void* scale_inv, int64_t ld_scale, int scale_dtype,
                void* y, int64_t ldy,
                int M, int N, int K,
                void* workspace, int64_t workspace_bytes,
                void* stream);

/* hs_int4_gemm / hs_fp8_gemm with a load-time tiled copy of the weight
 * (the "kernel-native layout" of the weight; same GPU branch of awq_linear /
 * fp8_linear, hydraserve/kernels/awq.py:25-75, hydraserve/kernels/fp8.py:24-97).
 * tiles: rows 16t..16t+15 of 128-wide K chunk c stored contiguously as tile
 * (t, c) at byte (c * N/16 + t) * TB.  INT4: TB = 1024, 16 rows x 16 int32
 * words, rows in order, nibbles paired as kernels/tiles.py describes
 * (packed.view(N/16, 16, K/128, 16).permute(2, 0, 1, 3)).  FP8: TB = 2048,
 * the 16 bytes of row r at K 64h + 16p .. +16 at byte 1024h + 16(16p + r)
 * of the tile (data.view(N/16, 16, K/128, 2, 4, 16).permute(2, 0, 3, 4, 1, 5)).
 * Requires N % 16 == 0 and K % 128 == 0 for the tiles to be read; the
 * row-major weight is still passed and used by the kernels that do not read
 * tiles (the tiles serve the tiled decode kernel at 1..64 rows, where one
 * load instruction then reads one contiguous tile, and the 256x256 prefill
 * kernel above that, whose loads then touch fewer cache lines).  Results are those of
 * the untiled entry points to the same bars. */
int hs_int4_gemm_tiled(const void* x, int64_t ldx,
                       const int32_t* packed, int64_t ld_packed, const int32_t* tiles,
                       const void* scale, int64_t ld_scale, int scale_dtype,
                       const int32_t* zero_point, int64_t ld_zero,
                       void* y, int64_t ldy,
                       int M, int N, int K, int group,
                       void* workspace, int64_t workspace_bytes,
                       void* stream);
int hs_fp8_gemm_tiled(const void* x, int64_t ldx,
                      const uint8_t* data, int64_t ld_data, const uint8_t* tiles,
                      const void* scale_inv, int64_t ld_scale, int scale_dtype,
                      void* y, int64_t ldy,
                      int M, int N, int K,
                      void* workspace, int64_t workspace_bytes,
                      void* stream);

/* out[N,K] = (q - z) * s rounded once to out_dtype (the dtype of the scale in
 * the reference).  GPU counterpart of dequantize_int4_weight
 * (hydraserve/kernels/awq.py:6-22); bit-exact. */
int hs_int4_dequant(const int32_t* packed, int64_t ld_packed,
                    const void* scale, int64_t ld_scale, int scale_dtype,
                    const int32_t* zero_point, int64_t ld_zero,
                    void* out, int64_t ld_out, int out_dtype,
                    int N, int K, int group, void* stream);

/* out[N,K] = decode(W) * cast(scale_inv, out_dtype), rounded to out_dtype.
 * GPU counterpart of dequantize_fp8_weight (hydraserve/kernels/fp8.py:6-21);
 * bit-exact. */
int hs_fp8_dequant(const uint8_t* data, int64_t ld_data,
                   const void* scale_inv, int64_t ld_scale, int scale_dtype,
                   void* out, int64_t ld_out, int out_dtype,
                   int N, int K, void* stream);

/* Measurement aid, no counterpart in the reference: reads `bytes` bytes
 * (a multiple of 16, 16-byte aligned) from src once with `blocks` workgroups
 * of 256 threads and writes one word per workgroup to sink (sink_bytes >=
 * 4 * blocks).  Its duration gives the streaming-read ceiling the decode
 * GEMMs are compared against. */
int hs_hbm_read_probe(const void* src, int64_t bytes, void* sink, int64_t sink_bytes, int blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HYDRASERVE_AMD_H */
