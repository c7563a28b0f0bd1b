// jules_hip_pjrt.hpp - ROCm PJRT client, device and executable on top of
// libjules_hip.so.
//
// The classes mirror the reference's PJRT interface (include/jules/PJRT.h):
//   DeviceBuffer   :46-73    DeviceEvent :78-87    PJRTExecutable :113-129
//   PJRTDevice     :145-170  PJRTClient  :195-233
// with the same class names, method names, argument meaning and return types,
// two substitutions: element types are jh_dtype (jules_hip.h) instead of
// jules::ScalarType::ScalarKind, and failures throw jules_hip::PJRTError
// instead of reporting through a DiagnosticsEngine.  The reference's
// PJRTClient::create("rocm", diag) falls back to the CPU client today
// (PJRT.cpp:1278-1284); an adapter there can return this client instead.
//
// Executables take the same program text as the reference's CPU executable
// (StableHLO in generic op form, `%r = "stablehlo.op"(%a, %b) {...} : ...`)
// and give the same results for the ops it interprets (elementwise, dot_general,
// reshape, transpose, reduce, constant), computed on the GPU.  The difference is
// stablehlo.custom_call, which the reference executes as a copy of its first
// operand (PJRT.cpp:491-499): here call_target_name is looked up in the kernel
// registry (jules_hip_lookup) and the kernel runs, so the extern_kernel ops
// KernelRoutingPass emits execute.  All work of one device is issued on that
// device's stream in program order.
#ifndef JULES_HIP_PJRT_HPP
#define JULES_HIP_PJRT_HPP

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "jules_hip.h"

namespace jules_hip {

/// A failure of a PJRT operation; status() is the jh_status it maps to.
class PJRTError : public std::runtime_error {
public:
    PJRTError(int status, const std::string& what) : std::runtime_error(what), status_(status) {}
    int status() const { return status_; }

private:
    int status_;
};

/// A buffer in device memory (PJRT.h:46-73).  Owns the memory unless it is a
/// view created by wrapDeviceMemory().
class DeviceBuffer {
public:
    virtual ~DeviceBuffer() = default;
    virtual size_t size() const = 0;                      // bytes
    virtual std::vector<int64_t> shape() const = 0;
    virtual jh_dtype elementType() const = 0;
    virtual void copyFromHost(const void* data, size_t size) = 0;
    virtual void copyToHost(void* data, size_t size) const = 0;
    virtual void* rawPointer() = 0;                       // device address
    virtual int deviceId() const = 0;
    virtual bool isHostBuffer() const = 0;                // false: device memory
};

/// Completion of work issued on a device stream (PJRT.h:78-87).
class DeviceEvent {
public:
    virtual ~DeviceEvent() = default;
    virtual void await() = 0;
    virtual bool isReady() const = 0;
};

/// A loaded program (PJRT.h:113-129).  execute() returns after the device is
/// done; executeAsync() returns the outputs at once, valid to read after the
/// event completes.  Outputs are every value the program produces, in program
/// order (PJRT.cpp:300-323).
class PJRTExecutable {
public:
    virtual ~PJRTExecutable() = default;
    virtual std::vector<std::shared_ptr<DeviceBuffer>>
    execute(const std::vector<std::shared_ptr<DeviceBuffer>>& inputs) = 0;
    virtual std::pair<std::vector<std::shared_ptr<DeviceBuffer>>, std::shared_ptr<DeviceEvent>>
    executeAsync(const std::vector<std::shared_ptr<DeviceBuffer>>& inputs) = 0;
    virtual std::string name() const = 0;
};

/// One GPU (PJRT.h:145-170).  kind() is "ROCM_GPU", vendor() "AMD".
class PJRTDevice {
public:
    virtual ~PJRTDevice() = default;
    virtual int id() const = 0;
    virtual std::string kind() const = 0;
    virtual std::string vendor() const = 0;
    virtual size_t availableMemory() const = 0;
    virtual std::shared_ptr<DeviceBuffer> allocateBuffer(const std::vector<int64_t>& shape,
                                                         jh_dtype elementType) = 0;
    virtual std::shared_ptr<PJRTExecutable> loadExecutable(const std::string& serializedProgram) = 0;
};

/// The client (PJRT.h:195-233): platform "rocm", one PJRTDevice per visible GPU.
class PJRTClient {
public:
    virtual ~PJRTClient() = default;
    /// "rocm" (or "gpu"); any other platform throws PJRTError(JH_ERR_UNSUPPORTED).
    static std::unique_ptr<PJRTClient> create(const std::string& platform);
    virtual std::string platform() const = 0;
    virtual size_t deviceCount() const = 0;
    virtual PJRTDevice* getDevice(size_t index) = 0;
    virtual PJRTDevice* getDefaultDevice() = 0;
    virtual std::shared_ptr<DeviceBuffer> allocateBuffer(const std::vector<int64_t>& shape,
                                                         jh_dtype elementType) = 0;
    virtual std::shared_ptr<PJRTExecutable> compileAndLoad(const std::string& serializedProgram) = 0;
    virtual void synchronizeAll() = 0;
    /// Stage i+1 takes stage i's outputs as inputs; all stages are issued on
    /// the device stream back to back (stream order replaces host waits), and
    /// the call returns once the last stage is done.
    virtual std::vector<std::shared_ptr<DeviceBuffer>>
    executePipeline(const std::vector<PJRTExecutable*>& stages,
                    const std::vector<std::shared_ptr<DeviceBuffer>>& inputs) = 0;
};

/// A non-owning DeviceBuffer over caller-owned device memory on `device`.
std::shared_ptr<DeviceBuffer> wrapDeviceMemory(void* data, const std::vector<int64_t>& shape,
                                               jh_dtype elementType, int device);

/// The op list a program parses into for `numInputs` inputs, one line per op
/// (`<buffer indices out> = <kind> <buffer indices in> [attributes]`); for
/// tests and debugging.  Needs no GPU.
std::string describeProgram(const std::string& serializedProgram, size_t numInputs);

}  // namespace jules_hip

#endif  // JULES_HIP_PJRT_HPP
