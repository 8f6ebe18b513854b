// Measured ceilings for the roofline (no counterpart in the reference): a sustained bf16 MFMA stream over every CU,
// against which the GEMM and attention kernels' achieved rates are read next to the spec-sheet 2.5 PFLOP/s.
//
// Each wave keeps 8 independent 32x32 fp32 accumulators and issues v_mfma_f32_32x32x16_bf16 back to back: with 8
// chains a chain's next MFMA comes 8 MFMAs after its previous one, past the instruction's latency, so the issue rate
// alone bounds the loop. The operands are the caller's (random N(0, 1) bf16 for a realistic clock: the engine clock
// under load depends on the operand bits; zeros show the difference):
//   lds = 0: 4 A and 2 B fragments held in registers for the whole loop (the MFMA issue rate alone);
//   lds = 1: every MFMA's fragments read from a 32 KB LDS block of the operands, a new 1 KB per fragment and step
//            (ds_read_b128, about 96 bytes per clock per CU at the full MFMA rate, as the GEMM main loops read),
//            the next step's reads issued before the current step's MFMAs.
#include "common.h"

namespace noise {

constexpr int kCalFrags = 6;         // 4 A + 2 B fragments per step, 8 MFMAs
constexpr int kCalLdsFrags = 32;     // 32 KB of LDS: 32 fragments of 64 lanes x 16 bytes

template <bool kLds>
__global__ __launch_bounds__(256, 2) void peak_mfma_kernel(const bf16x8* __restrict__ ops, int64_t n_frag_rows,
                                                          int iters, float* __restrict__ out) {
  __shared__ bf16x8 lds[kCalLdsFrags * 64];
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  f32x16 acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = f32x16{};
  if constexpr (!kLds) {
    // fragment f of this wave: 64-lane row (wave * 6 + f) mod n_frag_rows of the operand block
    bf16x8 f[kCalFrags];
#pragma unroll
    for (int j = 0; j < kCalFrags; ++j) f[j] = ops[((wave * kCalFrags + j) % n_frag_rows) * 64 + lane];
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[2 * i + j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], f[4 + j], acc[2 * i + j], 0, 0, 0);
    }
  } else {
    // the workgroup's 32 KB block: fragment rows (blockIdx.x * 32 + r) mod n_frag_rows
    for (int r = threadIdx.x >> 6; r < kCalLdsFrags; r += 4)
      lds[r * 64 + lane] = ops[(((int64_t)blockIdx.x * kCalLdsFrags + r) % n_frag_rows) * 64 + lane];
    __syncthreads();
    const int w = threadIdx.x >> 6;
    // two register sets: the 6 reads of one step are issued before the 8 MFMAs of the other set's step (the
    // scheduling groups pin that order), so the reads' latency runs behind the MFMAs
    bf16x8 fa[kCalFrags], fb[kCalFrags];
    auto read = [&](bf16x8 (&f)[kCalFrags], int step) {
#pragma unroll
      for (int j = 0; j < kCalFrags; ++j) f[j] = lds[((w * 8 + step * kCalFrags + j) & (kCalLdsFrags - 1)) * 64 + lane];
    };
    auto mfma = [&](const bf16x8 (&f)[kCalFrags]) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[2 * i + j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], f[4 + j], acc[2 * i + j], 0, 0, 0);
    };
    read(fa, 0);
    for (int it = 0; it < iters; it += 2) {
      read(fb, it + 1);
      mfma(fa);
      __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      __builtin_amdgcn_sched_barrier(0);
      read(fa, it + 2);
      mfma(fb);
      __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[k][r];
  out[wave * 64 + lane] = s;  // keeps every product live
}

}  // namespace noise

using namespace noise;

// Sustained MFMA stream: `workgroups` workgroups of 4 waves, each wave `iters` steps of 8
// v_mfma_f32_32x32x16_bf16 (32,768 FLOP each); ops bf16 [n_frag_rows, 64, 8] (n_frag_rows >= 32), out fp32
// [workgroups * 256] (each lane's sum of its accumulators). FLOPs = workgroups * 4 * iters * 8 * 32768.
extern "C" int noise_peak_mfma(const uint16_t* ops, int64_t n_frag_rows, int32_t iters, int32_t workgroups,
                               int32_t lds, float* out, void* stream) {
  NOISE_REQUIRE(ops && out, "NULL pointer argument");
  NOISE_REQUIRE(!lds || iters % 2 == 0, "the LDS mode runs steps in pairs: iters must be even");
  NOISE_REQUIRE(n_frag_rows >= kCalLdsFrags, "n_frag_rows = %lld: at least %d rows of 64 x 8 bf16",
                (long long)n_frag_rows, kCalLdsFrags);
  NOISE_REQUIRE(iters > 0 && workgroups > 0 && workgroups <= (1 << 20), "iters and workgroups must be positive");
  if (lds)
    hipLaunchKernelGGL(peak_mfma_kernel<true>, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream,
                       (const bf16x8*)ops, n_frag_rows, iters, out);
  else
    hipLaunchKernelGGL(peak_mfma_kernel<false>, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream,
                       (const bf16x8*)ops, n_frag_rows, iters, out);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}
