// Internal state of the C++ runtime shared by its translation units
// (sfg_decoder.cpp: compile / execute; sfg_package.cpp: .sfe packages): the
// libsfg_hip.so function table, device buffers and a plan's device state.
// Not installed; callers use sfg_decoder.hpp.
#pragma once

#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <filesystem>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "sfg_decoder.hpp"

namespace schedforge::hip {

inline void hip_check(hipError_t rc, const char* what) {
    if (rc != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(rc));
}

// ---------------------------------------------------------------- generator

// SplitMix64 and the per-tensor stream key of the synthetic-data generator
// (seed, tensor id): element i of a stream draws splitmix64(key + i).
inline std::uint64_t splitmix64(std::uint64_t x) {
    std::uint64_t z = x + 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

inline std::uint64_t stream_key(std::uint64_t seed, std::uint32_t tensor_id) {
    return splitmix64(splitmix64(seed) ^ (static_cast<std::uint64_t>(tensor_id) * 0xD1B54A32D192ED03ULL));
}

// ---------------------------------------------------------------- library

// Function table of libsfg_hip.so, resolved once per process.
class SfgHipLibrary {
public:
    decltype(&sfg_hip_abi_version) abi_version = nullptr;
    decltype(&sfg_hip_metadata_v1) metadata = nullptr;
    decltype(&sfg_hip_last_error) last_error = nullptr;
    decltype(&sfg_hip_device_info_v1) device_info = nullptr;
    decltype(&sfg_hip_target_info_v1) target_info = nullptr;
    decltype(&sfg_hip_pack_weight_v1) pack_weight = nullptr;
    decltype(&sfg_hip_quantize_weight_v1) quantize_weight = nullptr;
    decltype(&sfg_hip_preferred_weight_layout_v1) preferred_layout = nullptr;
    decltype(&sfg_hip_rope_table_host_v1) rope_table = nullptr;
    decltype(&sfg_hip_decoder_layer_workspace_v1) layer_workspace = nullptr;
    decltype(&sfg_hip_decoder_layer_v1) layer = nullptr;
    decltype(&sfg_hip_events_create_v1) events_create = nullptr;
    decltype(&sfg_hip_events_destroy_v1) events_destroy = nullptr;
    decltype(&sfg_hip_event_elapsed_v1) event_elapsed = nullptr;
    std::string path;

    explicit SfgHipLibrary(const std::filesystem::path& file) : path(file.string()) {
        handle_ = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
        if (!handle_) throw std::runtime_error(std::string("cannot load libsfg_hip.so: ") + dlerror());
        bind(abi_version, "sfg_hip_abi_version");
        bind(metadata, "sfg_hip_metadata_v1");
        bind(last_error, "sfg_hip_last_error");
        bind(device_info, "sfg_hip_device_info_v1");
        bind(target_info, "sfg_hip_target_info_v1");
        bind(pack_weight, "sfg_hip_pack_weight_v1");
        bind(quantize_weight, "sfg_hip_quantize_weight_v1");
        bind(preferred_layout, "sfg_hip_preferred_weight_layout_v1");
        bind(rope_table, "sfg_hip_rope_table_host_v1");
        bind(layer_workspace, "sfg_hip_decoder_layer_workspace_v1");
        bind(layer, "sfg_hip_decoder_layer_v1");
        bind(events_create, "sfg_hip_events_create_v1");
        bind(events_destroy, "sfg_hip_events_destroy_v1");
        bind(event_elapsed, "sfg_hip_event_elapsed_v1");
        const std::string meta = metadata();
        if (abi_version() != SFG_HIP_ABI_VERSION || meta.find("abi=1") == std::string::npos ||
            meta.find("arch=gfx950") == std::string::npos)
            throw std::runtime_error("libsfg_hip.so ABI or target mismatch: " + meta);
    }
    ~SfgHipLibrary() {
        if (handle_) dlclose(handle_);
    }
    SfgHipLibrary(const SfgHipLibrary&) = delete;
    SfgHipLibrary& operator=(const SfgHipLibrary&) = delete;

    // Status codes below 16 are the reference's std::invalid_argument class.
    void check(int rc, const char* what) const {
        if (rc == SFG_OK) return;
        const std::string message = std::string(what) + ": " + last_error();
        if (rc < SFG_ERR_DEVICE) throw std::invalid_argument(message);
        throw std::runtime_error(message);
    }

    // Address of an exported symbol, nullptr when absent.
    void* lookup(const std::string& name) const { return dlsym(handle_, name.c_str()); }

private:
    template <typename Fn>
    void bind(Fn& fn, const char* name) {
        fn = reinterpret_cast<Fn>(dlsym(handle_, name));
        if (!fn) throw std::runtime_error(std::string("libsfg_hip.so lacks ") + name);
    }
    void* handle_ = nullptr;
};

// The process-wide library for `requested` (empty: SFG_HIP_LIBRARY, else
// libsfg_hip.so beside this runtime), loaded and validated once.
std::shared_ptr<SfgHipLibrary> load_library(const std::filesystem::path& requested);

// ---------------------------------------------------------------- device state

struct DeviceBuffer {
    void* ptr = nullptr;
    std::size_t bytes = 0;
    DeviceBuffer() = default;
    explicit DeviceBuffer(std::size_t n) : bytes(n) {
        if (n) hip_check(hipMalloc(&ptr, n), "hipMalloc");
    }
    ~DeviceBuffer() {
        if (ptr) (void)hipFree(ptr);
    }
    DeviceBuffer(DeviceBuffer&& other) noexcept : ptr(other.ptr), bytes(other.bytes) {
        other.ptr = nullptr;
        other.bytes = 0;
    }
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept {
        std::swap(ptr, other.ptr);
        std::swap(bytes, other.bytes);
        return *this;
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    template <typename T>
    T* as() const { return static_cast<T*>(ptr); }
};

struct DecoderExecutablePlan::Device {
    std::shared_ptr<SfgHipLibrary> lib;
    int ordinal = 0;
    hipStream_t stream = nullptr;
    sfg_layer_desc desc{};
    sfg_layer_weights weights{};
    std::vector<std::pair<std::string, DeviceBuffer>> buffers;
    DeviceBuffer workspace;
    DeviceBuffer trace_ids, trace_weights;
    std::mutex mutex;  // one execution of a plan at a time (shared stream and workspace)

    ~Device() {
        buffers.clear();
        if (stream) (void)hipStreamDestroy(stream);
    }
    void* add(const std::string& name, std::size_t bytes) {
        buffers.emplace_back(name, DeviceBuffer(bytes));
        return buffers.back().second.ptr;
    }
    void upload(void* dst, const void* src, std::size_t bytes) {
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream), "hipMemcpyAsync");
    }
    void sync() { hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize"); }
};

// Shared by compile and package loading.
GpuTargetInfo query_target(const SfgHipLibrary& lib, int ordinal);
std::string describe_hardware(const SfgHipLibrary& lib, int ordinal);
// The layer descriptor of a plan (everything but the device pointers).
void fill_layer_desc(sfg_layer_desc& d, const DecoderConfig& c, const DecoderPlanPolicy& policy,
                     int pages_per_seq, int num_pages, bool use_routing_trace);
// Allocates and zeroes the layer's workspace for dev.desc; returns its size.
std::size_t allocate_workspace(DecoderExecutablePlan::Device& dev);

}  // namespace schedforge::hip
