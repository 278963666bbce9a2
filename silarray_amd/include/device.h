#pragma once
// Device selection, mirroring include/device.h:7-16 of the reference
// (Device, device_, gpu_pending_, use_cpu(), use_mps()) with use_gpu() added.
//
// This build is the GPU backend: float arithmetic always runs on the MI355X.
// use_cpu() is accepted so reference programs compile, but float evaluation
// in CPU mode throws (the reference's Accelerate backend is not part of this
// build); int and bool arrays, which the reference also handles on the host,
// work in either mode.

namespace sil {

enum class Device {
  GPU,
  CPU,
  MPS = GPU,  // the reference's name for its GPU device
};

inline Device device_ = Device::GPU;
inline bool gpu_pending_ = false;  // set by every kernel launch, cleared by flush

inline void use_gpu() { device_ = Device::GPU; }
inline void use_mps() { device_ = Device::GPU; }
inline void use_cpu() { device_ = Device::CPU; }

}  // namespace sil
