// A stand-alone gfx950 code object for the module surface of the C ABI
// (teeny_hip_module_load / _load_data / _get_function / teeny_hip_launch).
//
// The reference loads each compiled kernel as a module and launches it with
// a void** argument array (CudaProgram::try_from_ptx and
// CudaDevice::launch_with_packer, drivers/teeny-cuda/src/device/
// program.rs:327-390 and device/mod.rs:430-490).  This file is built with
// `hipcc --genco` into teenygrad_amd/teeny_example.hsaco, a code object an
// executor can load through that surface without the operator library.
//
//   y[i] = a * x[i] + y[i]  for i < n   (grid-stride, any launch shape)
#include <hip/hip_runtime.h>

extern "C" __global__ void teeny_example_axpy(float a, const float *__restrict__ x,
                                              float *__restrict__ y, int n) {
  const int stride = static_cast<int>(gridDim.x * blockDim.x);
  for (int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x); i < n; i += stride)
    y[i] = a * x[i] + y[i];
}
