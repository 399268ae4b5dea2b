// modify.cpp -- GpuTable insert (placeholder until the GPU modify kernels land).
#include "layers.hpp"

namespace nve_amd {

void GpuTable::insert(ExecutionContext&, int64_t, const void*, int64_t, int64_t, const void*) {
  NVE_NOT_IMPLEMENTED("GPU table insert is not available yet");
}

void GpuTable::insert_from_uvm(ExecutionContext&, int64_t, const void*) {
  NVE_NOT_IMPLEMENTED("GPU table insert is not available yet");
}

}  // namespace nve_amd
