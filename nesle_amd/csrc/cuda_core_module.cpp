// cuda_core_module.cpp -- nesle_amd._cuda_core_native, imported by
// nesle_amd/_cuda_core.py: the drop-in for the
// reference's pybind11 module nesle._cuda_core (cpp/bindings/cuda_module.cu).
//
// A thin layer over the C ABI of libnesle_hip.so (include/nesle_hip.h): it
// keeps the reference's Python surface -- CudaBatch constructors, step /
// step_device / step_stats / step_profile / reset_envs / views, and
// CudaDeviceArrayView with __cuda_array_interface__ and __dlpack__ -- and adds
// snapshot capture/export and full-state save/load.  Host-only C++ (no HIP
// types); compiled with g++ against pybind11 and linked to libnesle_hip.so.
//
// Lifetime: the batch handle is reference counted in the library.  The
// CudaBatch object, every CudaDeviceArrayView and every DLPack capsule hold
// their own reference, so device memory outlives whichever of them goes
// last (the reference ties views to the batch with keep_alive and a Python
// reference in the capsule, cuda_module.cu:63-97, 1639-1669).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/nesle_hip.h"

namespace py = pybind11;

namespace {

void check(int rc) {
    if (rc == NESLE_OK) return;
    const std::string msg = nesle_last_error();
    if (rc == NESLE_EINVAL) throw py::value_error(msg);
    throw std::runtime_error(msg);
}

// DLPack ABI (v0.8 layout, the one torch.utils.dlpack consumes).
struct DLDevice { std::int32_t device_type; std::int32_t device_id; };
struct DLDataType { std::uint8_t code; std::uint8_t bits; std::uint16_t lanes; };
struct DLTensor {
    void* data;
    DLDevice device;
    std::int32_t ndim;
    DLDataType dtype;
    std::int64_t* shape;
    std::int64_t* strides;
    std::uint64_t byte_offset;
};
struct DLManagedTensor {
    DLTensor dl_tensor;
    void* manager_ctx;
    void (*deleter)(DLManagedTensor* self);
};
constexpr std::int32_t kDLROCM = 10;
constexpr std::uint8_t kDLInt = 0, kDLUInt = 1, kDLFloat = 2;

struct Managed {
    DLManagedTensor t{};
    std::int64_t shape[4] = {0, 0, 0, 0};
    nesle_batch* owner = nullptr;
};

void managed_deleter(DLManagedTensor* self) {
    if (self == nullptr) return;
    auto* m = static_cast<Managed*>(self->manager_ctx);
    nesle_release(m->owner);  // plain C: safe without the GIL, on any thread
    delete m;
}

const char* typestr_of(std::int32_t dtype) {
    switch (dtype) {
        case NESLE_DTYPE_U8: return "|u1";
        case NESLE_DTYPE_F32: return "<f4";
        case NESLE_DTYPE_U32: return "<u4";
        case NESLE_DTYPE_U64: return "<u8";
        case NESLE_DTYPE_I64: return "<i8";
        default: return "|u1";
    }
}

DLDataType dl_dtype_of(std::int32_t dtype) {
    switch (dtype) {
        case NESLE_DTYPE_U8: return {kDLUInt, 8, 1};
        case NESLE_DTYPE_F32: return {kDLFloat, 32, 1};
        case NESLE_DTYPE_U32: return {kDLUInt, 32, 1};
        case NESLE_DTYPE_U64: return {kDLUInt, 64, 1};
        case NESLE_DTYPE_I64: return {kDLInt, 64, 1};
        default: return {kDLUInt, 8, 1};
    }
}

// Non-owning view of one device buffer of a batch (cuda_module.cu:114-183).
class DeviceArrayView {
public:
    DeviceArrayView(nesle_batch* batch, const nesle_view& v) : batch_(batch), v_(v) { nesle_retain(batch_); }
    DeviceArrayView(const DeviceArrayView& o) : batch_(o.batch_), v_(o.v_) { nesle_retain(batch_); }
    DeviceArrayView& operator=(const DeviceArrayView&) = delete;
    ~DeviceArrayView() { nesle_release(batch_); }

    py::dict cuda_array_interface() const {
        py::dict out;
        py::tuple shape(v_.ndim);
        for (int i = 0; i < v_.ndim; ++i) shape[i] = v_.shape[i];
        out["shape"] = shape;
        out["typestr"] = typestr_of(v_.dtype);
        out["data"] = py::make_tuple(reinterpret_cast<std::uintptr_t>(v_.data), false);
        out["version"] = 3;
        return out;
    }

    py::tuple dlpack_device() const { return py::make_tuple(kDLROCM, v_.device_id); }

    // The producer's stream is synchronised before hand-off, as the
    // reference does (cuda_module.cu:138-174); `stream` is accepted and unused.
    py::capsule dlpack(const py::object& /*stream*/) const {
        check(nesle_synchronize(batch_));
        auto* m = new Managed();
        for (int i = 0; i < v_.ndim; ++i) m->shape[i] = v_.shape[i];
        m->owner = batch_;
        nesle_retain(batch_);
        m->t.dl_tensor.data = v_.data;
        m->t.dl_tensor.device = DLDevice{kDLROCM, v_.device_id};
        m->t.dl_tensor.ndim = v_.ndim;
        m->t.dl_tensor.dtype = dl_dtype_of(v_.dtype);
        m->t.dl_tensor.shape = m->shape;
        m->t.dl_tensor.strides = nullptr;
        m->t.dl_tensor.byte_offset = 0;
        m->t.manager_ctx = m;
        m->t.deleter = managed_deleter;
        return py::capsule(&m->t, "dltensor", [](PyObject* cap) {
            // Only an unconsumed capsule still carries the "dltensor" name.
            if (PyCapsule_IsValid(cap, "dltensor")) {
                auto* t = static_cast<DLManagedTensor*>(PyCapsule_GetPointer(cap, "dltensor"));
                if (t != nullptr && t->deleter != nullptr) t->deleter(t);
            }
        });
    }

    std::uintptr_t ptr() const { return reinterpret_cast<std::uintptr_t>(v_.data); }
    py::tuple shape() const {
        py::tuple s(v_.ndim);
        for (int i = 0; i < v_.ndim; ++i) s[i] = v_.shape[i];
        return s;
    }

private:
    nesle_batch* batch_;
    nesle_view v_;
};

std::vector<std::uint8_t> bytes_vec(const py::bytes& b) {
    const std::string s = b;
    return {s.begin(), s.end()};
}

// Device pointer + dtype of an action tensor (torch tensor or any object with
// __cuda_array_interface__), following cuda_module.cu:259-308.
std::uintptr_t device_actions(const py::object& obj, std::uint32_t n, int* dtype) {
    if (py::hasattr(obj, "data_ptr") && py::hasattr(obj, "is_cuda")) {
        if (!obj.attr("is_cuda").cast<bool>()) throw py::value_error("expected CUDA actions, got a CPU tensor");
        if (py::hasattr(obj, "is_contiguous") && !obj.attr("is_contiguous")().cast<bool>())
            throw py::value_error("CUDA action tensor must be contiguous");
        const auto shape = obj.attr("shape").cast<py::tuple>();
        if (shape.size() != 1 || shape[0].cast<std::uint32_t>() != n)
            throw py::value_error("CUDA action tensor must have shape (" + std::to_string(n) + ",)");
        const auto dt = py::str(obj.attr("dtype")).cast<std::string>();
        if (dt == "torch.uint8") *dtype = NESLE_DTYPE_U8;
        else if (dt == "torch.int64") *dtype = NESLE_DTYPE_I64;
        else throw py::value_error("CUDA actions must have dtype torch.uint8 or torch.int64");
        return obj.attr("data_ptr")().cast<std::uintptr_t>();
    }
    if (!py::hasattr(obj, "__cuda_array_interface__"))
        throw py::value_error("expected a CUDA tensor/array exposing __cuda_array_interface__");
    const py::dict iface = obj.attr("__cuda_array_interface__").cast<py::dict>();
    const auto shape = iface["shape"].cast<py::tuple>();
    if (shape.size() != 1 || shape[0].cast<std::uint32_t>() != n)
        throw py::value_error("CUDA action array must have shape (" + std::to_string(n) + ",)");
    const auto ts = iface["typestr"].cast<std::string>();
    if (ts == "|u1" || ts == "<u1") *dtype = NESLE_DTYPE_U8;
    else if (ts == "<i8" || ts == "|i8") *dtype = NESLE_DTYPE_I64;
    else throw py::value_error("CUDA actions must be uint8 masks or int64 values already encoded as masks");
    return iface["data"].cast<py::tuple>()[0].cast<std::uintptr_t>();
}

// Device pointer of a one-byte-per-env tensor (uint8 or bool) of shape (n,).
std::uintptr_t device_bytes(const py::object& obj, std::uint32_t n, int* dtype) {
    *dtype = NESLE_DTYPE_U8;
    if (py::hasattr(obj, "data_ptr") && py::hasattr(obj, "is_cuda")) {
        if (!obj.attr("is_cuda").cast<bool>()) throw py::value_error("expected a CUDA tensor, got a CPU tensor");
        if (py::hasattr(obj, "is_contiguous") && !obj.attr("is_contiguous")().cast<bool>())
            throw py::value_error("mask tensor must be contiguous");
        const auto shape = obj.attr("shape").cast<py::tuple>();
        if (shape.size() != 1 || shape[0].cast<std::uint32_t>() != n)
            throw py::value_error("mask tensor must have shape (" + std::to_string(n) + ",)");
        const auto dt = py::str(obj.attr("dtype")).cast<std::string>();
        if (dt != "torch.uint8" && dt != "torch.bool") throw py::value_error("mask tensor must be uint8 or bool");
        return obj.attr("data_ptr")().cast<std::uintptr_t>();
    }
    if (!py::hasattr(obj, "__cuda_array_interface__"))
        throw py::value_error("expected a CUDA tensor/array exposing __cuda_array_interface__");
    const py::dict iface = obj.attr("__cuda_array_interface__").cast<py::dict>();
    const auto shape = iface["shape"].cast<py::tuple>();
    if (shape.size() != 1 || shape[0].cast<std::uint32_t>() != n)
        throw py::value_error("mask array must have shape (" + std::to_string(n) + ",)");
    const auto ts = iface["typestr"].cast<std::string>();
    if (ts != "|u1" && ts != "<u1" && ts != "|b1") throw py::value_error("mask array must be uint8 or bool");
    return iface["data"].cast<py::tuple>()[0].cast<std::uintptr_t>();
}

struct RewardSpec {
    std::uint32_t kind = NESLE_REWARD_SMB, x_lo = 0x86, x_hi = 0x6D, done_addr = 0, clip = 15;
    float time_penalty = 0.0f;
};

class CudaBatch {
public:
    CudaBatch(std::uint32_t num_envs, std::uint32_t frameskip, const py::bytes& rom, const RewardSpec& r,
              std::int32_t device, std::uint32_t max_instructions, bool frames) {
        nesle_config cfg;
        nesle_config_init(&cfg);
        cfg.num_envs = num_envs;
        cfg.frameskip = frameskip;
        cfg.max_instructions_per_frame = max_instructions;
        cfg.reward_kind = r.kind;
        cfg.x_lo = r.x_lo;
        cfg.x_hi = r.x_hi;
        cfg.done_addr = r.done_addr;
        cfg.clip = r.clip;
        cfg.time_penalty = r.time_penalty;
        cfg.device = device;
        cfg.frames = frames ? 1u : 0u;
        frames_ = frames;
        const auto bytes = bytes_vec(rom);
        check(nesle_create(&cfg, bytes.data(), bytes.size(), &h_));
        n_ = num_envs;
    }
    // The ROM-less synthetic batch, CudaBatch(num_envs, frameskip)
    // (cuda_module.cu:368-379): name "cuda".
    CudaBatch(std::uint32_t num_envs, std::uint32_t frameskip, std::int32_t device, bool frames) {
        nesle_config cfg;
        nesle_config_init(&cfg);
        cfg.num_envs = num_envs;
        cfg.frameskip = frameskip;
        cfg.device = device;
        cfg.frames = frames ? 1u : 0u;
        frames_ = frames;
        synthetic_ = true;
        check(nesle_create_synthetic(&cfg, &h_));
        n_ = num_envs;
    }
    CudaBatch(const CudaBatch&) = delete;
    CudaBatch& operator=(const CudaBatch&) = delete;
    ~CudaBatch() { nesle_release(h_); }

    void set_snapshots(const std::vector<py::bytes>& snaps, const std::vector<std::uint8_t>* levels) {
        std::vector<std::vector<std::uint8_t>> raw;
        std::vector<const std::uint8_t*> ptrs;
        std::vector<std::size_t> lens;
        for (const auto& s : snaps) raw.push_back(bytes_vec(s));
        for (const auto& r : raw) {
            ptrs.push_back(r.data());
            lens.push_back(r.size());
        }
        check(nesle_set_snapshots(h_, ptrs.data(), lens.data(), static_cast<std::uint32_t>(ptrs.size()),
                                  levels ? levels->data() : nullptr));
        has_snapshot_ = true;
    }

    DeviceArrayView view(int kind) const {
        nesle_view v{};
        check(nesle_get_view(h_, kind, &v));
        return DeviceArrayView(h_, v);
    }

    template <typename T>
    py::array_t<T> host(int kind, std::vector<py::ssize_t> shape) const {
        py::array_t<T> out(shape);
        check(nesle_copy_to_host(h_, kind, out.mutable_data(), static_cast<std::size_t>(out.nbytes())));
        return out;
    }

    void set_host_actions(const py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>& actions) {
        const auto v = actions.request();
        if (v.ndim != 1 || static_cast<std::uint32_t>(v.shape[0]) != n_)
            throw py::value_error("actions must have shape (num_envs,)");
        check(nesle_set_actions(h_, v.ptr, NESLE_DTYPE_U8, 0));
    }

    // reset(): power-on or snapshot reset of every console, then the RGB
    // frames of the re-seeded presentation snapshot (cuda_module.cu:469-479);
    // a batch without frames returns the RAM observation instead.
    py::array_t<std::uint8_t> reset() {
        check(nesle_reset(h_));
        return frames_ ? render() : ram();
    }

    // Host RGB frames [N, 240, 256, 3], re-rendered first
    // (cuda_module.cu:820-839).
    py::array_t<std::uint8_t> render() {
        check(nesle_render(h_, NESLE_FRAME_RGB));
        return host<std::uint8_t>(NESLE_VIEW_FRAME_RGB, {py::ssize_t(n_), 240, 256, 3});
    }

    // One render launch producing any of the device outputs.
    // live: draw live state by the reference CPU core's rules (ppu.hpp:
    // 213-545) instead of the presentation snapshot by the batched core's.
    void render_frames_device(bool rgb, bool palette, bool gray84, bool live) {
        const std::uint32_t outputs = (rgb ? NESLE_FRAME_RGB : 0u) | (palette ? NESLE_FRAME_PALETTE : 0u) |
                                      (gray84 ? NESLE_FRAME_GRAY84 : 0u) | (live ? NESLE_FRAME_LIVE : 0u);
        check(nesle_render(h_, outputs));
    }

    DeviceArrayView reset_device() {
        check(nesle_reset(h_));
        return view(NESLE_VIEW_RAM);
    }

    // step(actions, render_frame, copy_obs) (cuda_module.cu:533-592): one
    // env-step, a render when either flag is set, and the RGB frames as
    // "obs" when copy_obs (the RAM observation on a batch without frames).
    py::dict step(const py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>& actions,
                  bool render_frame, bool copy_obs) {
        set_host_actions(actions);
        check(nesle_step(h_, 0, 0));
        if (frames_ && (render_frame || copy_obs)) check(nesle_render(h_, NESLE_FRAME_RGB));
        py::dict out;
        if (copy_obs) {
            out["obs"] = frames_ ? host<std::uint8_t>(NESLE_VIEW_FRAME_RGB, {py::ssize_t(n_), 240, 256, 3}) : ram();
        }
        out["rewards"] = host<float>(NESLE_VIEW_REWARDS, {py::ssize_t(n_)});
        out["dones"] = host<std::uint8_t>(NESLE_VIEW_DONES, {py::ssize_t(n_)});
        return out;
    }

    py::dict step_device(const py::object& actions, bool auto_reset, bool synchronize) {
        int dtype = NESLE_DTYPE_U8;
        const auto ptr = device_actions(actions, n_, &dtype);
        check(nesle_set_actions(h_, reinterpret_cast<const void*>(ptr), dtype, 1));
        if (synthetic_) {
            // Without a ROM the reference's step_device() runs the reward
            // kernel alone: the actions are copied but move nothing
            // (cuda_module.cu:620-633).
            check(nesle_synthetic_step(h_, 0, auto_reset ? 1 : 0));
        } else {
            check(nesle_step(h_, auto_reset ? 1 : 0, 0));
        }
        // The action copy, the step and the fused reset are ordered on the
        // batch's stream, so only an explicit request synchronises (the
        // reference also synchronises after every auto-reset step,
        // cuda_module.cu:594-600, to keep its host action copy from racing
        // the reset kernel).
        if (synchronize) check(nesle_synchronize(h_));
        py::dict out;
        out["rewards"] = view(NESLE_VIEW_REWARDS);
        out["dones"] = view(NESLE_VIEW_DONES);
        out["ram"] = view(NESLE_VIEW_RAM);
        return out;
    }

    py::dict step_stats(const py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>& actions,
                        int mode) {
        set_host_actions(actions);
        check(nesle_step(h_, 0, mode));
        py::dict out;
        out["rewards"] = host<float>(NESLE_VIEW_REWARDS, {py::ssize_t(n_)});
        out["dones"] = host<std::uint8_t>(NESLE_VIEW_DONES, {py::ssize_t(n_)});
        out["instructions"] = host<std::uint64_t>(NESLE_VIEW_INSTRUCTIONS, {py::ssize_t(n_)});
        out["frames_completed"] = host<std::uint32_t>(NESLE_VIEW_FRAMES, {py::ssize_t(n_)});
        out["budget_hits"] = host<std::uint32_t>(NESLE_VIEW_BUDGET_HITS, {py::ssize_t(n_)});
        if (mode == 2) {
            out["opcode_counts"] = host<std::uint64_t>(NESLE_VIEW_OPCODES, {256});
            out["pc_counts"] = host<std::uint64_t>(NESLE_VIEW_PCS, {65536});
        }
        return out;
    }

    py::array_t<std::uint8_t> ram() const { return host<std::uint8_t>(NESLE_VIEW_RAM, {py::ssize_t(n_), 2048}); }
    py::array_t<std::uint8_t> oam() const { return host<std::uint8_t>(NESLE_VIEW_OAM, {py::ssize_t(n_), 256}); }

    void reset_envs(const py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>& mask) {
        const auto v = mask.request();
        if (v.ndim != 1 || static_cast<std::uint32_t>(v.shape[0]) != n_)
            throw py::value_error("mask must have shape (num_envs,)");
        check(nesle_reset_envs(h_, static_cast<const std::uint8_t*>(v.ptr), 0));
    }

    // Masked reset from a device mask (torch tensor or __cuda_array_interface__
    // object, uint8/bool, shape (num_envs,)), enqueued on the batch's stream.
    void reset_envs_device(const py::object& mask) {
        int dtype = NESLE_DTYPE_U8;
        const auto ptr = device_bytes(mask, n_, &dtype);
        check(nesle_reset_envs(h_, reinterpret_cast<const std::uint8_t*>(ptr), 1));
    }

    void poke_ram(std::uint16_t address, std::uint8_t value) { check(nesle_poke_ram(h_, address, value)); }

    // One RAM byte per console (host uint8 array of shape (num_envs,)).
    void poke_ram_envs(std::uint16_t address, const py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>& values) {
        const auto v = values.request();
        if (v.ndim != 1 || static_cast<std::uint32_t>(v.shape[0]) != n_)
            throw py::value_error("values must have shape (num_envs,)");
        check(nesle_poke_ram_envs(h_, address, static_cast<const std::uint8_t*>(v.ptr), 0));
    }

    py::bytes save_state(std::uint32_t env) const {
        std::string out(NESLE_STATE_BYTES, '\0');
        check(nesle_save_state(h_, env, reinterpret_cast<std::uint8_t*>(out.data())));
        return py::bytes(out);
    }

    void load_state(const py::bytes& state, const py::object& mask) {
        const auto raw = bytes_vec(state);
        std::vector<std::uint8_t> m;
        if (!mask.is_none()) {
            auto arr = mask.cast<py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>>();
            if (arr.ndim() != 1 || static_cast<std::uint32_t>(arr.shape(0)) != n_)
                throw py::value_error("mask must have shape (num_envs,)");
            m.assign(arr.data(), arr.data() + n_);
        }
        check(nesle_load_state(h_, raw.data(), raw.size(), mask.is_none() ? nullptr : m.data()));
    }

    void snapshot_capture(std::uint32_t env, std::uint32_t slot) {
        check(nesle_snapshot_capture(h_, env, slot));
        has_snapshot_ = true;
    }

    py::bytes snapshot_export(std::uint32_t slot) const {
        std::string out(NESLE_STATE_BYTES, '\0');
        check(nesle_snapshot_export(h_, slot, reinterpret_cast<std::uint8_t*>(out.data())));
        return py::bytes(out);
    }

    void set_env_levels(const py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>& levels) {
        if (levels.ndim() != 1 || static_cast<std::uint32_t>(levels.shape(0)) != n_)
            throw py::value_error("env_to_level must have shape (num_envs,)");
        check(nesle_set_env_levels(h_, levels.data()));
    }

    void synchronize() const { check(nesle_synchronize(h_)); }
    void set_timing(bool enable) { check(nesle_set_timing(h_, enable ? 1 : 0)); }
    py::tuple kernel_timing() const {
        double ms = 0.0;
        std::uint64_t n = 0;
        check(nesle_get_timing(h_, &ms, &n));
        return py::make_tuple(ms, n);
    }
    py::tuple kernel_timing_split() const {
        double ms = 0.0, reset_ms = 0.0;
        std::uint64_t n = 0;
        check(nesle_get_timing_split(h_, &ms, &reset_ms, &n));
        return py::make_tuple(ms, reset_ms, n);
    }
    void set_stream(std::uintptr_t stream) { check(nesle_set_stream(h_, reinterpret_cast<void*>(stream))); }

    std::uint32_t num_envs() const { return n_; }
    bool synthetic() const { return synthetic_; }
    std::uint32_t frameskip() const { return nesle_frameskip(h_); }
    std::uint32_t num_levels() const { return nesle_num_levels(h_); }
    bool has_snapshot() const { return has_snapshot_ && nesle_num_levels(h_) > 0; }
    bool frames() const { return frames_; }
    int device_id() const { return nesle_device_id(h_); }

private:
    nesle_batch* h_ = nullptr;
    std::uint32_t n_ = 0;
    bool has_snapshot_ = false;
    bool frames_ = true;
    bool synthetic_ = false;
};

RewardSpec reward_from_kwargs(const py::kwargs& kw) {
    RewardSpec r;
    if (kw.contains("reward")) {
        const auto spec = kw["reward"].cast<py::dict>();
        const auto kind = spec.contains("kind") ? spec["kind"].cast<std::string>() : std::string("smb");
        if (kind == "smb") {
            r.kind = NESLE_REWARD_SMB;
        } else if (kind == "x_delta") {
            r.kind = NESLE_REWARD_XDELTA;
        } else {
            throw py::value_error("reward kind must be 'smb' or 'x_delta'");
        }
        if (spec.contains("x_lo")) r.x_lo = spec["x_lo"].cast<std::uint32_t>();
        if (spec.contains("x_hi")) r.x_hi = spec["x_hi"].cast<std::uint32_t>();
        if (spec.contains("done_addr")) r.done_addr = spec["done_addr"].cast<std::uint32_t>();
        if (spec.contains("clip")) r.clip = spec["clip"].cast<std::uint32_t>();
        if (spec.contains("time_penalty")) r.time_penalty = spec["time_penalty"].cast<float>();
    }
    return r;
}

std::int32_t device_from_kwargs(const py::kwargs& kw) {
    return kw.contains("device") ? kw["device"].cast<std::int32_t>() : -1;
}

std::uint32_t budget_from_kwargs(const py::kwargs& kw) {
    return kw.contains("max_instructions_per_frame") ? kw["max_instructions_per_frame"].cast<std::uint32_t>() : 0u;
}

bool frames_from_kwargs(const py::kwargs& kw) { return kw.contains("frames") ? kw["frames"].cast<bool>() : true; }

}  // namespace

PYBIND11_MODULE(_cuda_core_native, m) {
    m.doc() = "MI355X NeSLE batch (HIP) -- drop-in for nesle._cuda_core";
    m.attr("STATE_BYTES") = NESLE_STATE_BYTES;
    m.attr("DLPACK_DEVICE_TYPE") = kDLROCM;

    py::class_<DeviceArrayView>(m, "CudaDeviceArrayView")
        .def_property_readonly("__cuda_array_interface__", &DeviceArrayView::cuda_array_interface)
        .def("__dlpack__", &DeviceArrayView::dlpack, py::arg("stream") = py::none())
        .def("__dlpack_device__", &DeviceArrayView::dlpack_device)
        .def_property_readonly("ptr", &DeviceArrayView::ptr)
        .def_property_readonly("shape", &DeviceArrayView::shape);

    m.def(
        "parse_fcs_state",
        [](const py::bytes& data) {
            const auto raw = bytes_vec(data);
            std::vector<std::uint8_t> b(NESLE_STATE_BYTES);
            check(nesle_parse_fcs(raw.data(), raw.size(), b.data()));
            auto u16 = [&](std::size_t o) { return static_cast<int>(b[o] | (b[o + 1] << 8)); };
            py::dict out;
            out["pc"] = u16(4);
            out["a"] = b[6]; out["x"] = b[7]; out["y"] = b[8]; out["sp"] = b[9]; out["p"] = b[10];
            out["cycles"] = 0;
            out["ppu_ctrl"] = b[32]; out["ppu_mask"] = b[33]; out["ppu_status"] = b[34];
            out["ppu_oam_addr"] = b[35]; out["ppu_open_bus"] = b[36]; out["ppu_read_buffer"] = b[37];
            out["ppu_x"] = b[42]; out["ppu_w"] = b[43]; out["ppu_v"] = u16(38); out["ppu_t"] = u16(40);
            auto slice = [&](std::size_t o, std::size_t n) { return py::bytes(reinterpret_cast<const char*>(b.data() + o), n); };
            out["cpu_ram"] = slice(80, 2048);
            out["prg_ram"] = slice(2128, 8192);
            out["nametable_ram"] = slice(10608, 2048);
            out["palette_ram"] = slice(10576, 32);
            out["oam"] = slice(10320, 256);
            return out;
        },
        py::arg("data"), "Parse an already-decompressed FCEUX FCS save state into a dict of fields.");

    m.def(
        "parse_ines_metadata",
        [](const py::bytes& data) {
            const auto raw = bytes_vec(data);
            nesle_rom_info info{};
            check(nesle_parse_ines(raw.data(), raw.size(), &info));
            py::dict out;
            out["prg_rom_size"] = info.prg_rom_size;
            out["chr_rom_size"] = info.chr_rom_size;
            out["mapper"] = info.mapper;
            out["submapper"] = info.submapper;
            static const char* kNt[] = {"vertical", "horizontal", "four_screen"};
            out["nametable_arrangement"] = kNt[info.nametable_arrangement % 3];
            out["has_trainer"] = info.has_trainer != 0;
            out["has_battery"] = info.has_battery != 0;
            out["is_nes2"] = info.is_nes2 != 0;
            return out;
        },
        py::arg("data"));

    py::class_<CudaBatch>(m, "CudaBatch")
        .def(py::init([](std::uint32_t num_envs, std::uint32_t frameskip, const py::kwargs& kw) {
                 return new CudaBatch(num_envs, frameskip, device_from_kwargs(kw), frames_from_kwargs(kw));
             }),
             py::arg("num_envs"), py::arg("frameskip"))
        .def(py::init([](std::uint32_t num_envs, std::uint32_t frameskip, const py::bytes& rom, const py::kwargs& kw) {
                 return new CudaBatch(num_envs, frameskip, rom, reward_from_kwargs(kw), device_from_kwargs(kw),
                                      budget_from_kwargs(kw), frames_from_kwargs(kw));
             }),
             py::arg("num_envs"), py::arg("frameskip"), py::arg("rom_bytes"))
        .def(py::init([](std::uint32_t num_envs, std::uint32_t frameskip, const py::bytes& rom, const py::bytes& snap,
                         const py::kwargs& kw) {
                 auto* b = new CudaBatch(num_envs, frameskip, rom, reward_from_kwargs(kw), device_from_kwargs(kw),
                                         budget_from_kwargs(kw), frames_from_kwargs(kw));
                 try {
                     b->set_snapshots({snap}, nullptr);
                 } catch (...) {
                     delete b;
                     throw;
                 }
                 return b;
             }),
             py::arg("num_envs"), py::arg("frameskip"), py::arg("rom_bytes"), py::arg("snapshot_bytes"))
        .def(py::init([](std::uint32_t num_envs, std::uint32_t frameskip, const py::bytes& rom,
                         const std::vector<py::bytes>& snaps,
                         const py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>& env_to_level,
                         const py::kwargs& kw) {
                 if (snaps.empty()) throw py::value_error("snapshot_bytes_list must contain at least one snapshot");
                 if (snaps.size() > 255) throw py::value_error("at most 255 snapshot levels supported per CudaBatch");
                 if (env_to_level.ndim() != 1 || static_cast<std::uint32_t>(env_to_level.shape(0)) != num_envs)
                     throw py::value_error("env_to_level must have shape (num_envs,)");
                 std::vector<std::uint8_t> levels(env_to_level.data(), env_to_level.data() + num_envs);
                 auto* b = new CudaBatch(num_envs, frameskip, rom, reward_from_kwargs(kw), device_from_kwargs(kw),
                                         budget_from_kwargs(kw), frames_from_kwargs(kw));
                 try {
                     b->set_snapshots(snaps, &levels);
                 } catch (...) {
                     delete b;
                     throw;
                 }
                 return b;
             }),
             py::arg("num_envs"), py::arg("frameskip"), py::arg("rom_bytes"), py::arg("snapshot_bytes_list"),
             py::arg("env_to_level"))
        .def("reset", &CudaBatch::reset)
        .def("reset_device", &CudaBatch::reset_device)
        .def("step", &CudaBatch::step, py::arg("actions"), py::arg("render_frame") = true, py::arg("copy_obs") = true)
        .def("step_device", &CudaBatch::step_device, py::arg("actions"), py::arg("auto_reset") = true,
             py::arg("synchronize") = true)
        .def("step_stats", [](CudaBatch& b, const py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>& a) {
                 return b.step_stats(a, 1);
             }, py::arg("actions"))
        .def("step_profile", [](CudaBatch& b, const py::array_t<std::uint8_t, py::array::c_style | py::array::forcecast>& a) {
                 return b.step_stats(a, 2);
             }, py::arg("actions"))
        .def("render", &CudaBatch::render)
        .def("render_device", [](CudaBatch& b) { b.render_frames_device(true, false, false, false); })
        .def("render_frames_device", &CudaBatch::render_frames_device, py::arg("rgb") = true,
             py::arg("palette") = false, py::arg("gray84") = false, py::arg("live") = false)
        .def("frames_device", [](const CudaBatch& b) { return b.view(NESLE_VIEW_FRAME_RGB); })
        .def("palette_frames_device", [](const CudaBatch& b) { return b.view(NESLE_VIEW_FRAME_PALETTE); })
        .def("gray84_device", [](const CudaBatch& b) { return b.view(NESLE_VIEW_GRAY84); })
        .def("ram", &CudaBatch::ram)
        .def("oam", &CudaBatch::oam)
        .def("ram_device", [](const CudaBatch& b) { return b.view(NESLE_VIEW_RAM); })
        .def("rewards_device", [](const CudaBatch& b) { return b.view(NESLE_VIEW_REWARDS); })
        .def("last_done_device", [](const CudaBatch& b) { return b.view(NESLE_VIEW_DONES); })
        .def("actions_device", [](const CudaBatch& b) { return b.view(NESLE_VIEW_ACTIONS); })
        .def("reset_envs", &CudaBatch::reset_envs, py::arg("mask"))
        .def("reset_envs_device", &CudaBatch::reset_envs_device, py::arg("mask"))
        .def("poke_ram", &CudaBatch::poke_ram, py::arg("address"), py::arg("value"))
        .def("poke_ram_envs", &CudaBatch::poke_ram_envs, py::arg("address"), py::arg("values"))
        .def("save_state", &CudaBatch::save_state, py::arg("env"))
        .def("load_state", &CudaBatch::load_state, py::arg("state"), py::arg("mask") = py::none())
        .def("snapshot_capture", &CudaBatch::snapshot_capture, py::arg("env"), py::arg("slot"))
        .def("snapshot_export", &CudaBatch::snapshot_export, py::arg("slot"))
        .def("set_env_levels", &CudaBatch::set_env_levels, py::arg("env_to_level"))
        .def("synchronize", &CudaBatch::synchronize)
        .def("set_timing", &CudaBatch::set_timing, py::arg("enable"))
        .def("kernel_timing", &CudaBatch::kernel_timing)
        .def("kernel_timing_split", &CudaBatch::kernel_timing_split)
        .def("set_stream", &CudaBatch::set_stream, py::arg("stream"))
        .def_property_readonly("name", [](const CudaBatch& b) { return std::string(b.synthetic() ? "cuda" : "cuda-console"); })
        .def_property_readonly("has_snapshot", &CudaBatch::has_snapshot)
        .def_property_readonly("frames", &CudaBatch::frames)
        .def_property_readonly("num_levels", &CudaBatch::num_levels)
        .def_property_readonly("num_envs", &CudaBatch::num_envs)
        .def_property_readonly("frameskip", &CudaBatch::frameskip)
        .def_property_readonly("device_id", &CudaBatch::device_id);
}
