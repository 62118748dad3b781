// dsv4_probe.hip - test-only library (libdsv4_probe.so): instructions of the
// gfx950 ISA that the product kernels rely on, run one tile or one code set at
// a time so the tests can pin their operand layouts and conversions against
// the reference's own decode. Nothing in the product library links or calls
// this; it is built beside the tests only.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

#define MX_FP8 0
#define MX_FP4 4

// Every FP4 code (both nibbles of bytes 0..255 through the MX convert with
// scale 1.0) and every E4M3 code (the OCP convert), as the GEMVs decode them.
__global__ void k_probe_converts(float *__restrict__ fp4_out, float *__restrict__ fp8_out) {
  const uint32_t t = threadIdx.x;  // 0..255
  const uint32_t word = t | (t << 8) | (t << 16) | (t << 24);
  const auto a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 0);
  fp4_out[2 * t] = a[0];
  fp4_out[2 * t + 1] = a[1];
  const auto b = __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
  fp8_out[t] = b[0];
}

static __device__ __forceinline__ v8i u4x2_to_v8i(uint4 a, uint4 b) {
  v8i r;
  r[0] = (int)a.x; r[1] = (int)a.y; r[2] = (int)a.z; r[3] = (int)a.w;
  r[4] = (int)b.x; r[5] = (int)b.y; r[6] = (int)b.z; r[7] = (int)b.w;
  return r;
}

// One 16x16 V_MFMA_SCALE_F32_16X16X128_F8F6F4 tile from row-major operands.
// A: [16][128] FP8 bytes or [16][64] packed FP4; B: [16][128] FP8 (one row per
// output column); scales [16][4] E8M0 codes. D: [16][16] row-major.
template <int AFMT>
__global__ void k_probe_mx(float *D, const uint8_t *A, const uint8_t *B, const uint8_t *sa,
                           const uint8_t *sb) {
  const int l = threadIdx.x, i = l % 16, kb = l / 16;
  uint4 a0, a1 = make_uint4(0, 0, 0, 0);
  if (AFMT == MX_FP4) {
    a0 = *reinterpret_cast<const uint4 *>(A + i * 64 + kb * 16);
  } else {
    a0 = *reinterpret_cast<const uint4 *>(A + i * 128 + kb * 16);
    a1 = *reinterpret_cast<const uint4 *>(A + i * 128 + 64 + kb * 16);
  }
  const uint4 b0 = *reinterpret_cast<const uint4 *>(B + i * 128 + kb * 16);
  const uint4 b1 = *reinterpret_cast<const uint4 *>(B + i * 128 + 64 + kb * 16);
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(u4x2_to_v8i(a0, a1),
                                                         u4x2_to_v8i(b0, b1), acc, AFMT, MX_FP8,
                                                         0, sa[i * 4 + kb], 0, sb[i * 4 + kb]);
  for (int v = 0; v < 4; ++v) D[(4 * kb + v) * 16 + i] = acc[v];
}

// One 16x16 V_MFMA_F32_16X16X32_BF16 tile: A [16][32], B [16][32] bf16 bits.
__global__ void k_probe_bf16(float *D, const uint16_t *A, const uint16_t *B) {
  const int l = threadIdx.x, i = l % 16, kb = l / 16;
  const uint4 a = *reinterpret_cast<const uint4 *>(A + i * 32 + kb * 8);
  const uint4 b = *reinterpret_cast<const uint4 *>(B + i * 32 + kb * 8);
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  for (int v = 0; v < 4; ++v) D[(4 * kb + v) * 16 + i] = acc[v];
}

static int launch_status(void) { return hipGetLastError() == hipSuccess ? 0 : -1; }

extern "C" {

// fp4_out: 512 floats (both nibbles of bytes 0..255); fp8_out: 256 floats.
int dsv4p_probe_converts(float *fp4_out, float *fp8_out, void *stream) {
  hipLaunchKernelGGL(k_probe_converts, dim3(1), dim3(256), 0, (hipStream_t)stream, fp4_out,
                     fp8_out);
  return launch_status();
}

// kind 0: FP4 x FP8 block-scaled, 1: FP8 x FP8 block-scaled, 2: BF16.
int dsv4p_probe_mfma(int kind, float *D, const void *A, const void *B, const uint8_t *sa,
                     const uint8_t *sb, void *stream) {
  hipStream_t st = (hipStream_t)stream;
  if (kind == 2)
    hipLaunchKernelGGL(k_probe_bf16, dim3(1), dim3(64), 0, st, D, (const uint16_t *)A,
                       (const uint16_t *)B);
  else if (kind == 0)
    hipLaunchKernelGGL(k_probe_mx<MX_FP4>, dim3(1), dim3(64), 0, st, D, (const uint8_t *)A,
                       (const uint8_t *)B, sa, sb);
  else if (kind == 1)
    hipLaunchKernelGGL(k_probe_mx<MX_FP8>, dim3(1), dim3(64), 0, st, D, (const uint8_t *)A,
                       (const uint8_t *)B, sa, sb);
  else
    return -2;
  return launch_status();
}

}  // extern "C"
