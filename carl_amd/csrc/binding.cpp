// binding.cpp - the `carl_amd._carl` Python module (pybind11).
//
// Same surface and error behaviour as the reference binding
// (python/carl.cu:18-989): DLPack inputs are validated completely - dtype,
// device (ROCm device 0), shape, contiguity, mask xor indices - before any
// state-changing call, raising TypeError / ValueError; outputs are
// non-owning DLPack views of environment buffers valid until the next call
// that repacks them.  Everything below the module is the C-ABI of
// include/carl_amd.h.
#include <hip/hip_runtime_api.h>
#include <pybind11/pybind11.h>

#include <cstdint>
#include <cstring>
#include <deque>
#include <initializer_list>
#include <optional>
#include <string>
#include <vector>

#include "../../include/carl_amd.h"

namespace py = pybind11;

namespace {

// ---- DLPack ABI (dlpack.h v0.x) ----
struct DLDevice { int32_t device_type; int32_t device_id; };
struct DLDataType { uint8_t code; uint8_t bits; uint16_t lanes; };
struct DLTensor {
    void* data;
    DLDevice device;
    int32_t ndim;
    DLDataType dtype;
    int64_t* shape;
    int64_t* strides;
    uint64_t byte_offset;
};
struct DLManagedTensor {
    DLTensor dl_tensor;
    void* manager_ctx;
    void (*deleter)(DLManagedTensor*);
};
constexpr int32_t kDLROCM = 10;
constexpr uint8_t kDLInt = 0, kDLFloat = 2, kDLBool = 6;

constexpr int kActPerCar = 7;
constexpr int kInternalSize = 19;

void check(int rc)
{
    if (rc == CARL_OK) return;
    const std::string msg = carl_last_error();
    if (rc == CARL_ERR_TYPE) throw py::type_error(msg);
    if (rc == CARL_ERR_VALUE) throw py::value_error(msg);
    throw std::runtime_error(msg);
}

py::capsule toCapsule(py::object obj, void* stream)
{
    if (py::isinstance<py::capsule>(obj)) return obj.cast<py::capsule>();
    return obj.attr("__dlpack__")(py::arg("stream") = reinterpret_cast<intptr_t>(stream)).cast<py::capsule>();
}

struct OwnedShape {
    int64_t shape[3];
};

void capsuleDeleter(PyObject* o)
{
    const char* name = PyCapsule_GetName(o);
    if (name && std::strcmp(name, "dltensor") == 0) {
        auto* t = static_cast<DLManagedTensor*>(PyCapsule_GetPointer(o, "dltensor"));
        if (t && t->deleter) t->deleter(t);
    }
}

py::object outputCapsule(carl_env* env, int id)
{
    void* data = nullptr;
    int64_t shape[3];
    int ndim = 0, dtype = 0;
    check(carl_env_buffer(env, id, &data, shape, &ndim, &dtype));
    auto* owned = new OwnedShape{ { shape[0], shape[1], shape[2] } };
    auto* t = new DLManagedTensor{};
    t->dl_tensor.data = data;
    t->dl_tensor.device = { kDLROCM, 0 };
    t->dl_tensor.ndim = ndim;
    t->dl_tensor.dtype = dtype == CARL_DTYPE_F32 ? DLDataType{ kDLFloat, 32, 1 }
                       : dtype == CARL_DTYPE_I32 ? DLDataType{ kDLInt, 32, 1 }
                                                 : DLDataType{ kDLBool, 8, 1 };
    t->dl_tensor.shape = owned->shape;
    t->dl_tensor.strides = nullptr;
    t->dl_tensor.byte_offset = 0;
    t->manager_ctx = owned;
    t->deleter = [](DLManagedTensor* self) {
        delete static_cast<OwnedShape*>(self->manager_ctx);
        delete self;
    };
    return py::capsule(t, "dltensor", capsuleDeleter);
}

struct TensorView {
    py::capsule capsule;
    DLTensor tensor;
    const void* data() const { return static_cast<const char*>(tensor.data) + tensor.byte_offset; }
};

// An empty simulation_indices tensor may have a null data pointer; the C-ABI
// reads a null index pointer as "every simulation", so an empty selection
// passes a dummy (never dereferenced) pointer instead.
const int64_t kNoIndex = 0;
const int64_t* selectionPointer(const TensorView& sel)
{
    const auto* p = static_cast<const int64_t*>(sel.data());
    return p ? p : &kNoIndex;
}

struct PendingInput {
    std::vector<py::object> inputs;
    hipEvent_t done = nullptr;
    explicit PendingInput(std::vector<py::object> in) : inputs(std::move(in))
    {
        if (hipEventCreateWithFlags(&done, hipEventDisableTiming) != hipSuccess)
            throw std::runtime_error("hipEventCreateWithFlags failed");
    }
    PendingInput(const PendingInput&) = delete;
    PendingInput& operator=(const PendingInput&) = delete;
    ~PendingInput()
    {
        if (done) (void)hipEventDestroy(done);
    }
};

class Env {
    carl_env* env_ = nullptr;
    int nSim_ = 0, nCars_ = 0;
    std::deque<PendingInput> pending_;

    void* stream() const { return carl_env_stream(env_); }

    void releaseInputs()
    {
        while (!pending_.empty()) {
            const hipError_t s = hipEventQuery(pending_.front().done);
            if (s == hipErrorNotReady) return;
            if (s != hipSuccess) throw std::runtime_error(hipGetErrorString(s));
            pending_.pop_front();
        }
    }

    static void validate(const DLTensor& t, const std::string& name, std::initializer_list<int64_t> shape, uint8_t code,
                         uint8_t bits)
    {
        if (t.dtype.code != code || t.dtype.bits != bits || t.dtype.lanes != 1)
            throw py::type_error(name + " has an invalid dtype");
        if (t.device.device_type != kDLROCM || t.device.device_id != 0)
            throw py::value_error(name + " must be on cuda:0");
        if (t.ndim != (int32_t)shape.size()) throw py::value_error(name + " has an invalid shape");
        int dim = 0;
        for (int64_t want : shape)
            if (t.shape[dim++] != want) throw py::value_error(name + " has an invalid shape");
        if (t.strides) {
            int64_t stride = 1;
            for (int i = t.ndim - 1; i >= 0; i--) {
                if (t.shape[i] > 1 && t.strides[i] != stride) throw py::value_error(name + " must be contiguous");
                stride *= t.shape[i];
            }
        }
    }

    TensorView view(py::object obj, const std::string& name, std::initializer_list<int64_t> shape, uint8_t code,
                    uint8_t bits) const
    {
        py::capsule cap = toCapsule(obj, stream());
        const auto* m = cap.get_pointer<DLManagedTensor>();
        if (!m) throw py::value_error("invalid DLPack tensor");
        const DLTensor t = m->dl_tensor;
        validate(t, name, shape, code, bits);
        return TensorView{ std::move(cap), t };
    }

    TensorView selection(py::object obj) const
    {
        py::capsule cap = toCapsule(obj, stream());
        const auto* m = cap.get_pointer<DLManagedTensor>();
        if (!m) throw py::value_error("invalid DLPack tensor");
        const DLTensor t = m->dl_tensor;
        if (t.dtype.code != kDLInt || t.dtype.bits != 64 || t.dtype.lanes != 1)
            throw py::type_error("simulation_indices must have dtype int64");
        if (t.device.device_type != kDLROCM || t.device.device_id != 0)
            throw py::value_error("simulation_indices must be on cuda:0");
        if (t.ndim != 1) throw py::value_error("simulation_indices must be one-dimensional");
        if (t.strides && t.strides[0] != 1) throw py::value_error("simulation_indices must be contiguous");
        if (t.shape[0] > nSim_) throw py::value_error("too many simulation_indices");
        return TensorView{ std::move(cap), t };
    }

    TensorView demoedView(py::object obj, const std::string& name, int n, bool& byteDemoed) const
    {
        py::capsule cap = toCapsule(obj, stream());
        const auto* m = cap.get_pointer<DLManagedTensor>();
        if (!m) throw py::value_error("invalid DLPack tensor");
        const DLTensor t = m->dl_tensor;
        byteDemoed = t.dtype.code == kDLBool && t.dtype.bits == 8;
        if (!byteDemoed && !(t.dtype.code == kDLInt && t.dtype.bits == 32))
            throw py::type_error(name + " must have dtype bool or int32");
        validate(t, name, { n, nCars_ }, t.dtype.code, t.dtype.bits);
        return TensorView{ std::move(cap), t };
    }

    TensorView actionData(py::object actions, bool continuous) const
    {
        py::capsule cap = toCapsule(actions, stream());
        const auto* m = cap.get_pointer<DLManagedTensor>();
        if (!m) throw py::value_error("invalid DLPack tensor");
        const DLTensor& t = m->dl_tensor;
        const std::string what = continuous ? "continuous actions" : "actions";
        const bool okType = continuous ? (t.dtype.code == kDLFloat && t.dtype.bits == 32 && t.dtype.lanes == 1)
                                       : (t.dtype.code == kDLInt && t.dtype.bits == 32 && t.dtype.lanes == 1);
        if (!okType) throw py::type_error(what + (continuous ? " must have dtype float32" : " must have dtype int32"));
        if (t.device.device_type != kDLROCM || t.device.device_id != 0)
            throw py::value_error(what + " must be on cuda:0");
        if (t.ndim != 3 || t.shape[0] != nSim_ || t.shape[1] != nCars_ || t.shape[2] != kActPerCar)
            throw py::value_error(what + " must have shape [n_sim, n_cars, 7]");
        if (t.strides && (t.strides[2] != 1 || t.strides[1] != kActPerCar || t.strides[0] != nCars_ * kActPerCar))
            throw py::value_error(what + " must be contiguous");
        return TensorView{ std::move(cap), t };
    }

    // The engine stream reads caller memory after the call returns; keep the
    // producer's tensors alive until that stream has passed this point, so a
    // temporary freed by the caller cannot be reused under a pending read.
    void holdUntilConsumed(std::vector<py::object> keep)
    {
        pending_.emplace_back(std::move(keep));
        if (hipEventRecord(pending_.back().done, (hipStream_t)stream()) != hipSuccess)
            throw std::runtime_error("hipEventRecord failed");
    }

public:
    Env(int nSim, int nBlue, int nOrange, int seed, int frameskip, bool invertOrange, bool normalize,
        bool previousControls)
    {
        if (frameskip < 1) throw py::value_error("frameskip must be at least 1");
        const int flags = (invertOrange ? CARL_FLAG_INVERT_ORANGE : 0) | (normalize ? CARL_FLAG_NORMALIZE : 0)
                        | (previousControls ? CARL_FLAG_PREVIOUS_CONTROLS : 0);
        check(carl_env_create(nSim, nBlue, nOrange, seed, frameskip, flags, &env_));
        nSim_ = nSim;
        nCars_ = nBlue + nOrange;
    }

    ~Env()
    {
        if (!env_) return;
        (void)carl_env_synchronize(env_);
        pending_.clear();
        carl_env_destroy(env_);
    }

    py::object step(py::object actions)
    {
        releaseInputs();
        const TensorView a = actionData(actions, false);
        check(carl_env_step(env_, CARL_ACTIONS_DISCRETE, a.data()));
        holdUntilConsumed({ a.capsule });
        return outputCapsule(env_, CARL_BUF_OBS);
    }

    py::object stepContinuous(py::object actions)
    {
        releaseInputs();
        const TensorView a = actionData(actions, true);
        check(carl_env_step(env_, CARL_ACTIONS_CONTINUOUS, a.data()));
        holdUntilConsumed({ a.capsule });
        return outputCapsule(env_, CARL_BUF_OBS);
    }

    void reset()
    {
        releaseInputs();
        check(carl_env_reset(env_));
    }

    void setBall(py::object position, py::object velocity, py::object angular, py::object indices)
    {
        int n = nSim_;
        std::optional<TensorView> sel;
        const int64_t* idx = nullptr;
        if (!indices.is_none()) {
            sel.emplace(selection(indices));
            idx = selectionPointer(*sel);
            n = (int)sel->tensor.shape[0];
        }
        const auto p = view(position, "position", { n, 3 }, kDLFloat, 32);
        const auto v = view(velocity, "velocity", { n, 3 }, kDLFloat, 32);
        const auto a = view(angular, "angular_velocity", { n, 3 }, kDLFloat, 32);
        check(carl_env_set_ball(env_, (const float*)p.data(), (const float*)v.data(), (const float*)a.data(), idx, n));
        check(carl_env_synchronize(env_));
    }

    void setCar(py::object position, py::object rotation, py::object velocity, py::object angular, py::object demoed,
                py::object boost, py::object internal, py::object indices)
    {
        int n = nSim_;
        std::optional<TensorView> sel;
        const int64_t* idx = nullptr;
        if (!indices.is_none()) {
            sel.emplace(selection(indices));
            idx = selectionPointer(*sel);
            n = (int)sel->tensor.shape[0];
        }
        const auto p = view(position, "position", { n, nCars_, 3 }, kDLFloat, 32);
        const auto r = view(rotation, "rotation", { n, nCars_, 4 }, kDLFloat, 32);
        const auto v = view(velocity, "velocity", { n, nCars_, 3 }, kDLFloat, 32);
        const auto a = view(angular, "angular_velocity", { n, nCars_, 3 }, kDLFloat, 32);
        bool byteDemoed = false;
        const auto d = demoedView(demoed, "demoed", n, byteDemoed);
        std::optional<TensorView> b, in;
        if (!boost.is_none()) b.emplace(view(boost, "boost", { n, nCars_ }, kDLFloat, 32));
        if (!internal.is_none()) in.emplace(view(internal, "internal_state", { n, nCars_, kInternalSize }, kDLFloat, 32));
        check(carl_env_set_car(env_, (const float*)p.data(), (const float*)r.data(), (const float*)v.data(),
                               (const float*)a.data(), d.data(), byteDemoed ? 1 : 0,
                               b ? (const float*)b->data() : nullptr, in ? (const float*)in->data() : nullptr, idx, n));
        check(carl_env_synchronize(env_));
    }

    void applyResetState(py::object bpos, py::object bvel, py::object bang, py::object cpos, py::object crot,
                         py::object cvel, py::object cang, py::object demoed, py::object boost, py::object internal,
                         py::object blue, py::object orange, py::object ticks, py::object indices, py::object mask)
    {
        releaseInputs();
        if (!mask.is_none() && !indices.is_none())
            throw py::value_error("specify reset_mask or simulation_indices, not both");
        int n = nSim_;
        std::optional<TensorView> sel, maskView;
        const int64_t* idx = nullptr;
        if (!indices.is_none()) {
            sel.emplace(selection(indices));
            idx = selectionPointer(*sel);
            n = (int)sel->tensor.shape[0];
        }
        if (!mask.is_none()) maskView.emplace(view(mask, "reset_mask", { nSim_ }, kDLBool, 8));
        // every input is validated before any state-changing call
        const auto bp = view(bpos, "ball_position", { n, 3 }, kDLFloat, 32);
        const auto bv = view(bvel, "ball_velocity", { n, 3 }, kDLFloat, 32);
        const auto ba = view(bang, "ball_angular_velocity", { n, 3 }, kDLFloat, 32);
        const auto cp = view(cpos, "car_position", { n, nCars_, 3 }, kDLFloat, 32);
        const auto cr = view(crot, "car_rotation", { n, nCars_, 4 }, kDLFloat, 32);
        const auto cv = view(cvel, "car_velocity", { n, nCars_, 3 }, kDLFloat, 32);
        const auto ca = view(cang, "car_angular_velocity", { n, nCars_, 3 }, kDLFloat, 32);
        bool byteDemoed = false;
        const auto dm = demoedView(demoed, "car_demoed", n, byteDemoed);
        std::optional<TensorView> bo, in, bl, orr, tk;
        if (!boost.is_none()) bo.emplace(view(boost, "car_boost", { n, nCars_ }, kDLFloat, 32));
        if (!internal.is_none())
            in.emplace(view(internal, "car_internal_state", { n, nCars_, kInternalSize }, kDLFloat, 32));
        const bool hasMatch = !blue.is_none();
        if (hasMatch != !orange.is_none() || hasMatch != !ticks.is_none())
            throw py::value_error("blue_score, orange_score and episode_ticks must be supplied together");
        if (hasMatch) {
            bl.emplace(view(blue, "blue_score", { n }, kDLInt, 32));
            orr.emplace(view(orange, "orange_score", { n }, kDLInt, 32));
            tk.emplace(view(ticks, "episode_ticks", { n }, kDLInt, 32));
        }
        if (n == 0) return;
        const uint8_t* m = maskView ? (const uint8_t*)maskView->data() : nullptr;
        std::vector<py::object> keep;
        if (m) {
            keep = { maskView->capsule, bp.capsule, bv.capsule, ba.capsule, cp.capsule,
                                             cr.capsule, cv.capsule, ca.capsule, dm.capsule };
            if (bo) keep.push_back(bo->capsule);
            if (in) keep.push_back(in->capsule);
            if (hasMatch) {
                keep.push_back(bl->capsule);
                keep.push_back(orr->capsule);
                keep.push_back(tk->capsule);
            }
        }
        check(carl_env_apply_reset(
            env_, (const float*)bp.data(), (const float*)bv.data(), (const float*)ba.data(), (const float*)cp.data(),
            (const float*)cr.data(), (const float*)cv.data(), (const float*)ca.data(), dm.data(), byteDemoed ? 1 : 0,
            bo ? (const float*)bo->data() : nullptr, in ? (const float*)in->data() : nullptr,
            bl ? (const int32_t*)bl->data() : nullptr, orr ? (const int32_t*)orr->data() : nullptr,
            tk ? (const int32_t*)tk->data() : nullptr, idx, n, m));
        if (m) {
            holdUntilConsumed(std::move(keep));
        } else {
            check(carl_env_synchronize(env_));
            pending_.clear();
        }
    }

    void setMatchState(py::object blue, py::object orange, py::object ticks, py::object indices)
    {
        int n = nSim_;
        std::optional<TensorView> sel;
        const int64_t* idx = nullptr;
        if (!indices.is_none()) {
            sel.emplace(selection(indices));
            idx = selectionPointer(*sel);
            n = (int)sel->tensor.shape[0];
        }
        const auto b = view(blue, "blue_score", { n }, kDLInt, 32);
        const auto o = view(orange, "orange_score", { n }, kDLInt, 32);
        const auto t = view(ticks, "episode_ticks", { n }, kDLInt, 32);
        check(carl_env_set_match(env_, (const int32_t*)b.data(), (const int32_t*)o.data(), (const int32_t*)t.data(),
                                 idx, n));
    }

    void resetBoostPads(py::object indices)
    {
        int n = nSim_;
        std::optional<TensorView> sel;
        const int64_t* idx = nullptr;
        if (!indices.is_none()) {
            sel.emplace(selection(indices));
            idx = selectionPointer(*sel);
            n = (int)sel->tensor.shape[0];
        }
        check(carl_env_reset_pads(env_, idx, n));
        check(carl_env_synchronize(env_));
    }

    py::object buffer(int id) { return outputCapsule(env_, id); }

    int param(int p) const
    {
        int v = 0;
        check(carl_env_get_param(env_, p, &v));
        return v;
    }
    void setParam(int p, int v) { check(carl_env_set_param(env_, p, v)); }

    uintptr_t streamHandle() const { return reinterpret_cast<uintptr_t>(stream()); }

    py::list actionNvec() const
    {
        py::list cars;
        for (int c = 0; c < nCars_; c++) {
            py::list nvec;
            for (int n : { 3, 3, 3, 2, 2, 3, 2 }) nvec.append(n);
            cars.append(nvec);
        }
        return cars;
    }

    // checkpoint hooks (no reference counterpart): raw persistent state words
    py::tuple exportState()
    {
        std::vector<uint32_t> car((size_t)CARL_CAR_FIELDS * nSim_ * nCars_), sim((size_t)CARL_SIM_FIELDS * nSim_);
        int tick = 0;
        check(carl_env_export_state(env_, car.data(), sim.data(), &tick));
        return py::make_tuple(py::bytes((const char*)car.data(), car.size() * 4),
                              py::bytes((const char*)sim.data(), sim.size() * 4), tick);
    }

    void importState(py::bytes car, py::bytes sim, int tick)
    {
        const std::string c = car, s = sim;
        if (c.size() != (size_t)CARL_CAR_FIELDS * nSim_ * nCars_ * 4 || s.size() != (size_t)CARL_SIM_FIELDS * nSim_ * 4)
            throw py::value_error("state buffers have the wrong size");
        check(carl_env_import_state(env_, (const uint32_t*)c.data(), (const uint32_t*)s.data(), tick));
    }

    void tick(py::object actions, int kind, int n)
    {
        releaseInputs();
        py::capsule cap = toCapsule(actions, stream());
        const auto* m = cap.get_pointer<DLManagedTensor>();
        if (!m) throw py::value_error("invalid DLPack tensor");
        const DLTensor& t = m->dl_tensor;
        if (t.device.device_type != kDLROCM) throw py::value_error("actions must be on cuda:0");
        int64_t count = 1;
        for (int i = 0; i < t.ndim; i++) count *= t.shape[i];
        const int64_t want = (int64_t)nSim_ * nCars_ * (kind == CARL_ACTIONS_DIRECT ? 8 : 7);
        if (count != want || t.dtype.bits != 32) throw py::value_error("actions have the wrong size");
        check(carl_env_tick(env_, kind, static_cast<const char*>(t.data) + t.byte_offset, n));
        holdUntilConsumed({ cap });
    }

    void resetDones() { check(carl_env_reset_dones(env_)); }
    void synchronize() { check(carl_env_synchronize(env_)); }
    void enableTiming(bool on, bool ticks, bool packing, bool stages)
    {
        const int flags = (ticks ? CARL_TIME_TICKS : 0) | (packing ? CARL_TIME_PACKING : 0)
                          | (stages ? CARL_TIME_STAGES : 0);
        check(carl_env_enable_timing(env_, on ? flags : 0));
    }
    py::dict stageTiming()
    {
        double us[CARL_STAGES], last[CARL_STAGES + 1], spanUs = 0.0, launchUs = 0.0;
        int ticks = 0;
        check(carl_env_stage_timing(env_, us, last, &spanUs, &launchUs, &ticks));
        py::dict stages, critical;
        for (int s = 0; s < CARL_STAGES; s++) {
            stages[py::str(carl_stage_name(s))] = us[s];
            critical[py::str(carl_stage_name(s))] = last[s];
        }
        critical["start delay"] = last[CARL_STAGES];
        py::dict out;
        out["stages"] = stages;
        out["last_workgroup"] = critical;
        out["span_us"] = spanUs;
        out["launch_us"] = launchUs;
        out["ticks"] = ticks;
        return out;
    }
    py::dict tickTiming()
    {
        double ms[CARL_TICK_KERNELS];
        int launches[CARL_TICK_KERNELS];
        check(carl_env_tick_timing(env_, ms, launches));
        py::dict out;
        for (int k = 0; k < CARL_TICK_KERNELS; k++)
            if (launches[k] > 0) out[py::str(carl_tick_kernel_name(k))] = py::make_tuple(ms[k], launches[k]);
        return out;
    }
};

}  // namespace

PYBIND11_MODULE(_carl, m)
{
    m.doc() = "CARL step engine for AMD Instinct MI355X (HIP)";

    const int nvec[7] = { 3, 3, 3, 2, 2, 3, 2 };
    const float low[7] = { -1.f, -1.f, -1.f, 0.f, 0.f, -1.f, 0.f };
    py::tuple actionNvec(7), lowT(7), highT(7);
    int offsets[8] = { 0 };
    for (int f = 0; f < 7; f++) {
        actionNvec[f] = nvec[f];
        lowT[f] = low[f];
        highT[f] = 1.f;
        offsets[f + 1] = offsets[f] + nvec[f];
    }
    m.attr("ACTION_NVECS") = actionNvec;
    m.attr("ACTION_LOGITS") = offsets[7];
    m.attr("CONTINUOUS_ACTION_LOW") = lowT;
    m.attr("CONTINUOUS_ACTION_HIGH") = highT;
    // action fields: horizontal, vertical, throttle, powerslide, boost, air roll, jump
    auto nonNeutral = [&](int f) { return py::slice(py::int_(offsets[f] + 1), py::int_(offsets[f] + nvec[f]), py::none()); };
    m.attr("ACTION_PITCH_LOGITS") = nonNeutral(1);
    m.attr("ACTION_AIR_ROLL_LOGITS") = nonNeutral(5);
    m.attr("ACTION_POWERSLIDE_LOGIT") = offsets[3] + 1;
    m.attr("ACTION_BOOST_LOGIT") = offsets[4] + 1;
    m.attr("ACTION_JUMP_LOGIT") = offsets[6] + 1;

    // observation layout (reference include/Cuda/DLPack.h:60-107)
    const int OBS_POS = 0, OBS_VEL = 3, OBS_ANG = 6, OBS_FORWARD = 9, OBS_UP = 12, OBS_BOOST = 15;
    const int OBS_BALL = OBS_FORWARD, OBS_PER_CAR = 21;
    m.attr("OBS_VECTOR_SIZE") = 3;
    m.attr("OBS_POS") = OBS_POS;
    m.attr("OBS_VEL") = OBS_VEL;
    m.attr("OBS_ANG") = OBS_ANG;
    m.attr("OBS_FORWARD") = OBS_FORWARD;
    m.attr("OBS_UP") = OBS_UP;
    m.attr("OBS_BOOST") = OBS_BOOST;
    m.attr("OBS_ON_GROUND") = 16;
    m.attr("OBS_DEMOED") = 17;
    m.attr("OBS_HAS_FLIPPED") = 18;
    m.attr("OBS_HAS_DOUBLE_JUMPED") = 19;
    m.attr("OBS_IS_BOOSTING") = 20;
    m.attr("STATE_BALL_TOUCH") = 21;
    m.attr("OBS_BALL") = OBS_BALL;
    m.attr("OBS_PER_CAR") = OBS_PER_CAR;
    m.attr("STATE_PER_CAR") = 22;
    m.attr("NUM_BOOST_PADS") = 34;
    m.attr("OBS_BOOST_PADS") = 68;
    m.attr("OBS_RELATIVE_EGO_BALL") = 6;
    m.attr("OBS_RELATIVE_PER_OTHER_CAR") = 6;
    m.attr("OBS_RELATIVE_GOALS") = 6;
    m.attr("OBS_EGO_DODGE") = 2;
    m.attr("OBS_EGO_BOOST_INDEX") = OBS_BALL + OBS_BOOST;
    m.attr("OBS_EGO_ON_GROUND_INDEX") = OBS_BALL + 16;
    m.attr("OBS_EGO_FLIP_INDEX") = -2 - 5;
    m.attr("OBS_EGO_CONTROLLER") = 5;
    m.attr("OBS_PREVIOUS_CONTROLS") = 8;
    m.attr("OBS_CONTROLLER_VERSION") = 3;
    m.attr("CAR_INTERNAL_SIZE") = kInternalSize;
    m.attr("OBS_EGO_DODGE_TIME_INDEX") = -2 - 5 + 1;

    m.attr("PHYS_TICKS_PER_SECOND") = 120;
    m.attr("PHYS_DT") = 1.f / 120;
    m.attr("DOUBLEJUMP_MAX_DELAY") = 1.25f;
    m.attr("REGULATION_TICKS") = 5 * 60 * 120;
    m.attr("OBS_POSITION_SCALE") = py::make_tuple(4108.f, 6000.f, 2076.f);
    m.attr("BALL_MAX_SPEED") = 6000.f;
    m.attr("BALL_MAX_ANG_SPEED") = 6.f;
    m.attr("CAR_MAX_SPEED") = 2300.f;
    m.attr("CAR_MAX_ANG_SPEED") = 5.5f;
    m.attr("BOOST_MAX") = 100.f;
    const float pads[34][3] = {
        { -3584.f, 0.f, 73.f }, { 3584.f, 0.f, 73.f }, { -3072.f, 4096.f, 73.f }, { 3072.f, 4096.f, 73.f },
        { -3072.f, -4096.f, 73.f }, { 3072.f, -4096.f, 73.f },
        { 0.f, -4240.f, 70.f }, { -1792.f, -4184.f, 70.f }, { 1792.f, -4184.f, 70.f }, { -940.f, -3308.f, 70.f },
        { 940.f, -3308.f, 70.f }, { 0.f, -2816.f, 70.f }, { -3584.f, -2484.f, 70.f }, { 3584.f, -2484.f, 70.f },
        { -1788.f, -2300.f, 70.f }, { 1788.f, -2300.f, 70.f }, { -2048.f, -1036.f, 70.f }, { 0.f, -1024.f, 70.f },
        { 2048.f, -1036.f, 70.f }, { -1024.f, 0.f, 70.f }, { 1024.f, 0.f, 70.f }, { -2048.f, 1036.f, 70.f },
        { 0.f, 1024.f, 70.f }, { 2048.f, 1036.f, 70.f }, { -1788.f, 2300.f, 70.f }, { 1788.f, 2300.f, 70.f },
        { -3584.f, 2484.f, 70.f }, { 3584.f, 2484.f, 70.f }, { 0.f, 2816.f, 70.f }, { -940.f, 3308.f, 70.f },
        { 940.f, 3308.f, 70.f }, { -1792.f, 4184.f, 70.f }, { 1792.f, 4184.f, 70.f }, { 0.f, 4240.f, 70.f },
    };
    py::tuple padT(34);
    for (int p = 0; p < 34; p++) padT[p] = py::make_tuple(pads[p][0], pads[p][1], pads[p][2]);
    m.attr("BOOST_PAD_POSITIONS") = padT;

    py::class_<Env>(m, "Env")
        .def(py::init<int, int, int, int, int, bool, bool, bool>(), py::arg("n_sim"), py::arg("n_blue"),
             py::arg("n_orange"), py::arg("seed"), py::arg("frameskip") = 1, py::arg("invert_orange") = true,
             py::arg("normalize") = false, py::arg("previous_controls") = false)
        .def("step", &Env::step, py::arg("actions"))
        .def("step_continuous", &Env::stepContinuous, py::arg("actions"))
        .def("reset", &Env::reset)
        .def("apply_reset_state", &Env::applyResetState, py::arg("ball_position"), py::arg("ball_velocity"),
             py::arg("ball_angular_velocity"), py::arg("car_position"), py::arg("car_rotation"),
             py::arg("car_velocity"), py::arg("car_angular_velocity"), py::arg("car_demoed"),
             py::arg("car_boost") = py::none(), py::arg("car_internal_state") = py::none(),
             py::arg("blue_score") = py::none(), py::arg("orange_score") = py::none(),
             py::arg("episode_ticks") = py::none(), py::arg("simulation_indices") = py::none(),
             py::arg("reset_mask") = py::none())
        .def("set_ball", &Env::setBall, py::arg("position"), py::arg("velocity"), py::arg("angular_velocity"),
             py::arg("simulation_indices") = py::none())
        .def("set_car", &Env::setCar, py::arg("position"), py::arg("rotation"), py::arg("velocity"),
             py::arg("angular_velocity"), py::arg("demoed"), py::arg("boost") = py::none(),
             py::arg("internal_state") = py::none(), py::arg("simulation_indices") = py::none())
        .def("get_obs", [](Env& e) { return e.buffer(CARL_BUF_OBS); })
        .def("get_transition_obs", [](Env& e) { return e.buffer(CARL_BUF_TRANSITION_OBS); })
        .def("get_state", [](Env& e) { return e.buffer(CARL_BUF_STATE); })
        .def("get_transition_state", [](Env& e) { return e.buffer(CARL_BUF_TRANSITION_STATE); })
        .def("get_rewards", [](Env& e) { return e.buffer(CARL_BUF_REWARDS); })
        .def("get_dones", [](Env& e) { return e.buffer(CARL_BUF_DONES); })
        .def("set_match_state", &Env::setMatchState, py::arg("blue_score"), py::arg("orange_score"),
             py::arg("episode_ticks"), py::arg("simulation_indices") = py::none())
        .def("reset_boost_pads", &Env::resetBoostPads, py::arg("simulation_indices") = py::none())
        .def("get_score_difference", [](Env& e) { return e.buffer(CARL_BUF_SCORE_DIFFERENCE); })
        .def("get_episode_ticks", [](Env& e) { return e.buffer(CARL_BUF_EPISODE_TICKS); })
        .def("get_transition_score_difference", [](Env& e) { return e.buffer(CARL_BUF_TRANSITION_SCORE_DIFFERENCE); })
        .def("get_transition_episode_ticks", [](Env& e) { return e.buffer(CARL_BUF_TRANSITION_EPISODE_TICKS); })
        .def("get_overtime", [](Env& e) { return e.buffer(CARL_BUF_OVERTIME); })
        .def("get_transition_overtime", [](Env& e) { return e.buffer(CARL_BUF_TRANSITION_OVERTIME); })
        .def_property("max_ticks", nullptr, [](Env& e, int v) { e.setParam(CARL_PARAM_MAX_TICKS, v); })
        .def_property("overtime_timeout_ticks", nullptr,
                      [](Env& e, int v) { e.setParam(CARL_PARAM_OVERTIME_TIMEOUT_TICKS, v); })
        .def_property("no_touch_timeout_ticks", nullptr,
                      [](Env& e, int v) { e.setParam(CARL_PARAM_NO_TOUCH_TIMEOUT_TICKS, v); })
        .def_property("frameskip", [](Env& e) { return e.param(CARL_PARAM_FRAMESKIP); },
                      [](Env& e, int v) { e.setParam(CARL_PARAM_FRAMESKIP, v); })
        .def_property("tick_streams", [](Env& e) { return e.param(CARL_PARAM_TICK_STREAMS); },
                      [](Env& e, int v) { e.setParam(CARL_PARAM_TICK_STREAMS, v); })
        .def_property("contact_screen", [](Env& e) { return e.param(CARL_PARAM_CONTACT_SCREEN); },
                      [](Env& e, int v) { e.setParam(CARL_PARAM_CONTACT_SCREEN, v); })
        .def_property("tick_window", [](Env& e) { return e.param(CARL_PARAM_TICK_WINDOW); },
                      [](Env& e, int v) { e.setParam(CARL_PARAM_TICK_WINDOW, v); })
        .def_property_readonly("tick_window_launch", [](Env& e) { return e.param(CARL_PARAM_TICK_WINDOW_LAUNCH); })
        .def_property("tick_balance", [](Env& e) { return e.param(CARL_PARAM_TICK_BALANCE); },
                      [](Env& e, int v) { e.setParam(CARL_PARAM_TICK_BALANCE, v); })
        .def_property_readonly("tick_balanced_launch",
                               [](Env& e) { return e.param(CARL_PARAM_TICK_BALANCED_LAUNCH) != 0; })
        .def_property_readonly("obs_dim", [](Env& e) { return e.param(CARL_PARAM_OBS_DIM); })
        .def_property_readonly("act_dim", [](Env& e) { return e.param(CARL_PARAM_ACT_DIM); })
        .def_property_readonly("action_nvec", &Env::actionNvec)
        .def_property_readonly("n_sim", [](Env& e) { return e.param(CARL_PARAM_N_SIM); })
        .def_property_readonly("n_cars", [](Env& e) { return e.param(CARL_PARAM_N_CARS); })
        .def_property_readonly("stream", &Env::streamHandle)
        // engine extensions (not in the reference binding)
        .def("export_state", &Env::exportState)
        .def("import_state", &Env::importState, py::arg("car_state"), py::arg("sim_state"), py::arg("tick_count"))
        .def("tick", &Env::tick, py::arg("actions"), py::arg("kind"), py::arg("n_ticks") = 1)
        .def("get_actions", [](Env& e) { return e.buffer(CARL_BUF_ACTIONS); })
        .def("get_continuous_actions", [](Env& e) { return e.buffer(CARL_BUF_CONTINUOUS_ACTIONS); })
        .def("reset_dones", &Env::resetDones)
        .def("synchronize", &Env::synchronize)
        .def("enable_tick_timing", &Env::enableTiming, py::arg("enable") = true, py::arg("ticks") = true,
             py::arg("packing") = false, py::arg("stages") = false)
        .def("tick_timing", &Env::tickTiming)
        .def("stage_timing", &Env::stageTiming)
        .def_property_readonly("tick_count", [](Env& e) { return e.param(CARL_PARAM_TICK_COUNT); })
        .def_property_readonly("native_arena", [](Env& e) { return e.param(CARL_PARAM_NATIVE_ARENA) != 0; });
}
