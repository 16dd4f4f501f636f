// Runs the library's device fp32 -> bf16 conversion (f32_to_bf16_rne of
// cudalm-agent_amd/csrc/hip_common.h, the one every kernel's output goes
// through) over the fp32 bit patterns of an input file and writes the
// 16-bit results: bf16_round_check IN OUT (raw uint32 in, raw uint16 out).
// tests/test_gpu_bf16_round.py compares them with the oracle's integer
// round-to-nearest-even form.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "hip_common.h"

__global__ void convert(const uint32_t* in, uint16_t* out, size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n)
    out[i] = static_cast<uint16_t>(cudalm_hip::f32_to_bf16_rne(__builtin_bit_cast(float, in[i])));
}

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  FILE* f = fopen(argv[1], "rb");
  if (!f) return 3;
  std::vector<uint32_t> h;
  uint32_t v;
  while (fread(&v, 4, 1, f) == 1) h.push_back(v);
  fclose(f);
  const size_t n = h.size();
  uint32_t* din = nullptr;
  uint16_t* dout = nullptr;
  if (hipMalloc(&din, n * 4) != hipSuccess || hipMalloc(&dout, n * 2) != hipSuccess) return 4;
  if (hipMemcpy(din, h.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess) return 5;
  hipLaunchKernelGGL(convert, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, 0, din,
                     dout, n);
  std::vector<uint16_t> o(n);
  if (hipMemcpy(o.data(), dout, n * 2, hipMemcpyDeviceToHost) != hipSuccess) return 6;
  hipFree(din);
  hipFree(dout);
  FILE* g = fopen(argv[2], "wb");
  if (!g || fwrite(o.data(), 2, n, g) != n) return 7;
  fclose(g);
  printf("converted %zu\n", n);
  return 0;
}
