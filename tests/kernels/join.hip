// Test kernel of the host-entry contract test (tests/test_entry_contract.py): a multi-parameter
// kernel (three pointers and an int, as a hand-written or externally compiled kernel would take
// them) whose result pins the argument order: output = 0.625 * first + 0.375 * second.
#include <hip/hip_runtime.h>

extern "C" __global__ void join(const float *first, const float *second, float *output, int size) {
  for (int i = int(blockIdx.x * blockDim.x + threadIdx.x); i < size; i += int(gridDim.x * blockDim.x))
    output[i] = __fmaf_rn(second[i], 0.375f, first[i] * 0.625f);
}
