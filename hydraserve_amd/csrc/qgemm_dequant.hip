// Materialising dequantizers: the GPU side of dequantize_int4_weight
// (hydraserve/kernels/awq.py:6-22) and dequantize_fp8_weight
// (hydraserve/kernels/fp8.py:6-21).  The GEMMs never call these; they exist so
// the drop-in keeps the reference's oracle functions on device tensors, and so
// the in-register decode paths can be checked bit-for-bit on the GPU.
#include "qgemm_common.h"

namespace hsq {

enum OutDtype { OUT_BF16 = 0, OUT_F16 = 1, OUT_F32 = 2 };

__device__ __forceinline__ float round_to(float v, int odt) {
  if (odt == OUT_BF16) return __uint_as_float(static_cast<uint32_t>(to_bf16_bits(v)) << 16);
  if (odt == OUT_F16) return __half2float(__float2half_rn(v));
  return v;
}

__device__ __forceinline__ void store_out(void* out, int64_t idx, float v, int odt) {
  if (odt == OUT_BF16) {
    reinterpret_cast<uint16_t*>(out)[idx] = to_bf16_bits(v);
  } else if (odt == OUT_F16) {
    reinterpret_cast<__half*>(out)[idx] = __float2half_rn(v);
  } else {
    reinterpret_cast<float*>(out)[idx] = v;
  }
}

// One thread per packed word: 8 consecutive K of one row.
// out[n, k] = round_out((q - z) * s); (q - z) * s is exact in fp32.
__global__ void int4_dequant_kernel(const uint32_t* packed, int64_t ldw, const void* scale, int64_t lds, int sdt,
                                    const int32_t* zero, int64_t ldz, void* out, int64_t ldo, int odt, int N, int K,
                                    int group) {
  const int kw = (K + 7) >> 3;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(N) * kw) return;
  const int n = static_cast<int>(idx / kw), wi = static_cast<int>(idx % kw);
  const uint32_t w = packed[n * ldw + wi];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = wi * 8 + e;
    if (k >= K) break;
    const int g = k / group;
    const float s = load_scale_rt(scale, n * lds + g, sdt);
    const uint32_t zw = static_cast<uint32_t>(zero[(n >> 3) * ldz + g]);
    const int z = static_cast<int>((zw >> ((n & 7) * 4)) & 0xFu);
    const int q = static_cast<int>((w >> (4 * e)) & 0xFu);
    store_out(out, n * ldo + k, static_cast<float>(q - z) * s, odt);
  }
}

// One thread per weight byte.  out = round_out(decode(b) * round_out(s)):
// the scale is cast to the output dtype first, as fp8.py:20-21 does.
__global__ void fp8_dequant_kernel(const uint8_t* w, int64_t ldw, const void* scale, int64_t lds, int sdt, void* out,
                                   int64_t ldo, int odt, int N, int K) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(N) * K) return;
  const int n = static_cast<int>(idx / K), k = static_cast<int>(idx % K);
  const uint32_t b = w[n * ldw + k];
  const float v = __builtin_amdgcn_cvt_pk_f32_fp8(b, false)[0];
  const float s = round_to(load_scale_rt(scale, (n >> 7) * lds + (k >> 7), sdt), odt);
  store_out(out, n * ldo + k, v * s, odt);
}

hipError_t launch_int4_dequant(const uint32_t* packed, int64_t ldw, const void* scale, int64_t lds, int sdt,
                               const int32_t* zero, int64_t ldz, void* out, int64_t ldo, int odt, int N, int K,
                               int group, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(N) * ((K + 7) >> 3);
  if (total == 0) return hipSuccess;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(int4_dequant_kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), 0, stream, packed, ldw,
                     scale, lds, sdt, zero, ldz, out, ldo, odt, N, K, group);
  return hipGetLastError();
}

hipError_t launch_fp8_dequant(const uint8_t* w, int64_t ldw, const void* scale, int64_t lds, int sdt, void* out,
                              int64_t ldo, int odt, int N, int K, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(N) * K;
  if (total == 0) return hipSuccess;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(fp8_dequant_kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), 0, stream, w, ldw, scale,
                     lds, sdt, out, ldo, odt, N, K);
  return hipGetLastError();
}

}  // namespace hsq
