// The ATen current stream of a device as a raw hipStream_t, for the library's `stream`
// arguments (the reference's bridges call c10::cuda::getCurrentCUDAStream; on ROCm builds
// of libtorch the same stream is c10::hip::getCurrentHIPStream).
#include <c10/hip/HIPStream.h>

extern "C" void* mi355x_sys_current_stream(int device) {
  return c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream();
}
