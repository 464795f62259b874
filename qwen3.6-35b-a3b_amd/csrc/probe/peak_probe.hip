// Peak probes for the roofline figures of bench.py (measurement infrastructure, built into its own
// libmoe_peak_probe.so; the MoE library does not link it). The method follows the reference's own
// probes (tools/bw_probe_hip.cpp: a grid-stride 16-byte read of a large buffer, best over a
// launch-shape sweep; tools/gemm_peak.cpp: the matrix instruction's throughput with operands in
// registers), written for gfx950:
//   - probe_hbm_read: every lane streams 16-byte loads, four in flight per iteration, over a buffer
//     the caller makes far larger than the 256 MB MALL, so the bytes come from HBM; the loaded
//     words are folded into one value that is stored only if it equals a sentinel the data never
//     produces, which keeps every load alive.
//   - probe_mfma_f16: every wave issues v_mfma_f32_32x32x16_f16 (the prefill GEMMs' instruction)
//     on register operands, four independent accumulators per wave so that issue, not the
//     accumulator dependency, bounds it; each MFMA is 32 * 32 * 16 * 2 = 32768 FLOP.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) k_probe_read(const u32x4_t* __restrict__ p, size_t n16,
                                                    uint32_t* __restrict__ sink) {
  const size_t step = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * step < n16; i += 4 * step) {
    const u32x4_t a = __builtin_nontemporal_load(p + i);
    const u32x4_t b = __builtin_nontemporal_load(p + i + step);
    const u32x4_t c = __builtin_nontemporal_load(p + i + 2 * step);
    const u32x4_t d = __builtin_nontemporal_load(p + i + 3 * step);
    acc ^= (a.x + b.y) ^ (c.z + d.w) ^ (a.w ^ b.x ^ c.y ^ d.z) ^ (a.y + a.z + b.z + b.w + c.x + c.w + d.x + d.y);
  }
  for (; i < n16; i += step) {
    const u32x4_t a = p[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

__global__ void __launch_bounds__(256) k_probe_mfma(int iters, float* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  f16x8_t a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (_Float16)(0.001f * (float)(lane + j));
    b[j] = (_Float16)(0.002f * (float)(lane - j));
  }
  f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
  if (s == 1234.5f) sink[0] = s;
}

extern "C" {

// One read pass over `bytes` (a multiple of 16) of a device buffer: `blocks` workgroups of 256
// lanes. Returns 0, or the HIP error code of the launch.
int probe_hbm_read(const void* buf, size_t bytes, int blocks, void* sink, void* stream) {
  if (!buf || !sink || bytes % 16 || blocks <= 0) return -1;
  hipLaunchKernelGGL(k_probe_read, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const u32x4_t*>(buf), bytes / 16, reinterpret_cast<uint32_t*>(sink));
  return (int)hipGetLastError();
}

// `blocks` workgroups of 4 waves, each wave issuing 4 * iters MFMAs (32768 FLOP each).
int probe_mfma_f16(int blocks, int iters, void* sink, void* stream) {
  if (!sink || blocks <= 0 || iters <= 0) return -1;
  hipLaunchKernelGGL(k_probe_mfma, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters,
                     reinterpret_cast<float*>(sink));
  return (int)hipGetLastError();
}

}  // extern "C"
