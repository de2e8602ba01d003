// VALU issue rates of gfx950 per instruction form, for the cycle model of the
// LUMA step kernels.  Each kernel runs one instruction form (inline asm, so
// the compiler cannot fold it) in 8 independent chains per lane, all
// operands in VGPRs; the occupancy is fixed at 3 or 4 waves per SIMD through
// the dynamic LDS allocation.  Prints wave instructions per clock per CU,
// taking the clock as 2.4 GHz.
//
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         luma_amd/bench/valu_rates.hip -o /tmp/valu_rates && /tmp/valu_rates
//
// Every access stays in bounds: each workgroup writes its 256 results at
// out[blockIdx.x * 256 + threadIdx.x] (blocks * 256 elements allocated), and
// the LDS write is a never-taken branch inside the allocation.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>

#define N_IT 2048

template <typename V>
__device__ __forceinline__ V in_vgpr(V x) { asm("" : "+v"(x)); return x; }

#define KU(NAME, ASM)                                                           \
  __global__ __launch_bounds__(256) void NAME(uint32_t *out, uint32_t a0) {     \
    extern __shared__ uint32_t lds[];                                           \
    const uint32_t a = in_vgpr(a0), b = in_vgpr(0x3f400000u), c = in_vgpr(3u); \
    uint32_t v[8];                                                              \
    _Pragma("unroll") for (int j = 0; j < 8; ++j) v[j] = 0x3f800000u + 4096u * (threadIdx.x + j); \
    for (int i = 0; i < N_IT; ++i) {                                            \
      _Pragma("unroll") for (int j = 0; j < 8; ++j) asm volatile(ASM : "+v"(v[j]) : "v"(a), "v"(b), "v"(c)); \
    }                                                                           \
    uint32_t s = 0;                                                             \
    _Pragma("unroll") for (int j = 0; j < 8; ++j) s ^= v[j];                    \
    if (s == 12345u) lds[threadIdx.x] = s;                                      \
    out[blockIdx.x * 256 + threadIdx.x] = s;                                    \
  }

KU(k_fma3, "v_fma_f32 %0, %0, %1, %2")
KU(k_fmac, "v_fmac_f32 %0, %1, %2")
KU(k_fmamk, "v_fmamk_f32 %0, %0, 0x3dfbe76d, %1")
KU(k_fma_inl, "v_fma_f32 %0, %0, %1, 0.5")
KU(k_mul, "v_mul_f32 %0, %0, %1")
KU(k_mul_abs, "v_mul_f32_e64 %0, |%0|, %1")
KU(k_add, "v_add_f32 %0, %0, %1")
KU(k_sub_abs, "v_sub_f32_e64 %0, %1, |%0|")
KU(k_med3, "v_med3_f32 %0, %0, %1, %2")
KU(k_max, "v_max_f32 %0, %0, %1")
KU(k_andor, "v_and_or_b32 %0, %0, %1, %2")
KU(k_lshlor, "v_lshl_or_b32 %0, %0, %3, %1")
KU(k_xor, "v_xor_b32 %0, %0, %1")
KU(k_or3, "v_or3_b32 %0, %0, %1, %2")
KU(k_and, "v_and_b32 %0, %0, %1")
KU(k_and_lit, "v_and_b32 %0, 0x7fffffff, %0")
KU(k_shr, "v_lshrrev_b32 %0, 3, %0")
KU(k_addu, "v_add_u32 %0, %0, %1")
KU(k_bfe, "v_bfe_i32 %0, %0, 0, 16")
KU(k_cvt_f_i, "v_cvt_f32_i32 %0, %0")
KU(k_cvt_i_f, "v_cvt_i32_f32 %0, %0")
KU(k_cvt_f_u, "v_cvt_f32_u32 %0, %0")
KU(k_cvt_u8, "v_cvt_f32_ubyte1 %0, %0")
KU(k_fract, "v_fract_f32 %0, %0")
KU(k_floor, "v_floor_f32 %0, %0")
KU(k_mant, "v_frexp_mant_f32 %0, %0")
KU(k_fexp, "v_frexp_exp_i32_f32 %0, %0")
KU(k_exp, "v_exp_f32 %0, %0")
KU(k_log, "v_log_f32 %0, %0")
KU(k_sqrt, "v_sqrt_f32 %0, %0")
KU(k_rcp, "v_rcp_f32 %0, %0")
KU(k_cndmask, "v_cndmask_b32 %0, %0, %1, vcc")
KU(k_dpp, "v_mov_b32_dpp %0, %0 row_shr:1 row_mask:0xf bank_mask:0xf")

__global__ __launch_bounds__(256) void k_mad64(uint32_t *out, uint32_t a0) {
  extern __shared__ uint32_t lds[];
  const uint32_t a = in_vgpr(a0);
  uint64_t v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = 0x3f800000u + 4096u * (threadIdx.x + j);
  for (int i = 0; i < N_IT; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint64_t cy;
      const uint32_t x = (uint32_t)v[j] ^ (uint32_t)(v[j] >> 32);
      asm volatile("v_mad_u64_u32 %0, %1, %2, %3, 0" : "=v"(v[j]), "=s"(cy) : "v"(x), "v"(a));
    }
  }
  uint32_t s = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) s ^= (uint32_t)v[j];
  if (s == 12345u) lds[threadIdx.x] = s;
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

typedef void (*Kern)(uint32_t *, uint32_t);
struct Case { const char *name; Kern k; };

int main() {
  const Case cases[] = {
    {"v_fma_f32 v,v,v", k_fma3}, {"v_fmac_f32", k_fmac}, {"v_fmamk_f32", k_fmamk},
    {"v_fma_f32 v,v,0.5", k_fma_inl}, {"v_mul_f32", k_mul}, {"v_mul_f32 |v|", k_mul_abs},
    {"v_add_f32", k_add}, {"v_sub_f32 v,|v|", k_sub_abs}, {"v_med3_f32", k_med3},
    {"v_max_f32", k_max}, {"v_and_or_b32", k_andor}, {"v_lshl_or_b32", k_lshlor},
    {"v_xor_b32", k_xor}, {"v_or3_b32", k_or3}, {"v_and_b32", k_and},
    {"v_and_b32 lit", k_and_lit}, {"v_lshrrev_b32", k_shr}, {"v_add_u32", k_addu},
    {"v_bfe_i32", k_bfe}, {"v_cvt_f32_i32", k_cvt_f_i}, {"v_cvt_i32_f32", k_cvt_i_f},
    {"v_cvt_f32_u32", k_cvt_f_u}, {"v_cvt_f32_ubyte1", k_cvt_u8}, {"v_fract_f32", k_fract},
    {"v_floor_f32", k_floor}, {"v_frexp_mant_f32", k_mant}, {"v_frexp_exp_i32", k_fexp},
    {"v_exp_f32", k_exp}, {"v_log_f32", k_log}, {"v_sqrt_f32", k_sqrt}, {"v_rcp_f32", k_rcp},
    {"v_cndmask_b32 vcc", k_cndmask}, {"v_mov_b32_dpp", k_dpp}, {"v_mad_u64_u32", k_mad64},
  };
  const int blocks = 256 * 32;
  uint32_t *dbuf;
  if (hipMalloc(&dbuf, sizeof(uint32_t) * blocks * 256) != hipSuccess) return 1;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
  printf("wave-instructions per clock per CU at 2.4 GHz\n");
  for (const Case &cs : cases) {
    printf("%-20s", cs.name);
    for (int wps = 3; wps <= 4; ++wps) {
      const size_t lds = (160 * 1024) / wps - 256;
      hipLaunchKernelGGL(cs.k, dim3(blocks), dim3(256), lds, 0, dbuf, 0x3f7fbe77u);
      hipError_t le = hipGetLastError();
      if (le != hipSuccess) { printf(" launch error %s\n", hipGetErrorString(le)); return 2; }
      if (hipDeviceSynchronize() != hipSuccess) return 3;
      hipEventRecord(e0, 0);
      for (int r = 0; r < 3; ++r) hipLaunchKernelGGL(cs.k, dim3(blocks), dim3(256), lds, 0, dbuf, 0x3f7fbe77u);
      hipEventRecord(e1, 0);
      if (hipEventSynchronize(e1) != hipSuccess) return 4;
      float ms;
      hipEventElapsedTime(&ms, e0, e1);
      ms /= 3;
      const double wave_instr = (double)blocks * 4 * 8.0 * N_IT;
      printf("  %dw: %.2f", wps, wave_instr / (ms * 1e-3) / 256 / 2.4e9);
    }
    printf("\n");
  }
  hipFree(dbuf);
  return 0;
}
