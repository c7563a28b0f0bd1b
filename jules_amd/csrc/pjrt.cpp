// pjrt.cpp - ROCm PJRT client / device / executable (include/jules_hip_pjrt.hpp)
// and its C ABI (jules_hip_pjrt_* in include/jules_hip.h).
//
// The executable interprets the same StableHLO text as the reference's CPU
// executable (lib/PJRT.cpp, CPUTensorInterpreter :169-858) with the same
// parse rules and op semantics, on device buffers and the device's stream:
//   parse   one regex pass in text order (:348-500); %argI are buffers 0..n-1,
//           every matched op takes the next buffer index, an operand name not
//           defined yet takes a fresh index that nothing writes; an empty
//           program is one copy of buffer 0 (:197-205)
//   attrs   result shape (:505-541), transpose permutation (:545-564),
//           reduce dimensions (:567-594), constant values (:462-484)
//   run     an op whose operands were never written is skipped (:606-610 and
//           each execute*); binary/unary/transpose/reduce run as kernels of
//           pjrt_ops.hip; dot_general runs the fp32 GEMM of gemm_f32.hip
//           (the reference calls cblas_sgemm, :662-700) with the reference's
//           M/K/N rule; reshape and copy are device copies
//   outputs every written buffer with index >= #inputs, in index order; none:
//           copies of the inputs (:300-323)
// Differences, all deliberate:
//   - stablehlo.custom_call runs the registry kernel named by its
//     call_target_name (jules_hip_lookup; "gelu", the target StableHLO
//     lowering gives jules.gelu, resolves to fusedGelu), with its
//     backend_config and the result types written after "->"; the reference
//     copies operand 0 (:491-499).  `%r:N = "stablehlo.custom_call"(...)` with
//     uses `%r#i` gives multi-result calls (fusedCrossEntropyLoss).
//   - A program is parsed once per input count (the reference parses on the
//     first call only and reuses that parse for any later input count).
//   - Where the reference would read out of bounds (a transpose or reduce
//     whose data is not its shape's size, a dot_general operand smaller than
//     M*K or K*N, an invalid permutation) the executable throws PJRTError.
//   - Built-in ops need fp32 buffers (the reference reinterprets any buffer as
//     floats, :935-946); custom calls take whatever dtypes their kernel takes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <regex>
#include <sstream>

#include "jules_hip.h"
#include "jules_hip_pjrt.hpp"
#include "launch.hpp"

namespace jh {
int set_last_error(int status, const std::string& message);
}

namespace jules_hip {
namespace {

[[noreturn]] void fail(int status, const std::string& msg) { throw PJRTError(status, msg); }

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(JH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

size_t dtype_size(jh_dtype t) {
    switch (t) {
        case JH_F32: return 4;
        case JH_BF16: return 2;
        case JH_I8: return 1;
        case JH_I32: return 4;
    }
    fail(JH_ERR_DTYPE, "unknown element type");
}

int64_t elements(const std::vector<int64_t>& shape) {
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d < 0) fail(JH_ERR_SHAPE, "negative dimension");
        n *= d;
    }
    return n;
}

// ---------------------------------------------------------------------------
// Program: the parsed op list.
// ---------------------------------------------------------------------------
struct POp {
    enum Kind { Binary, Unary, MatMul, Constant, Reshape, Transpose, Reduce, CustomCall, Copy };
    Kind kind = Copy;
    int sub = 0;                         // PjOp of binary / unary ops
    std::string opname;
    std::vector<int> ins, outs;
    std::vector<int64_t> shape;          // reshape: parsed result shape (may be empty)
    std::vector<int64_t> perm, dims;     // transpose, reduce
    std::vector<float> data;             // constant
    std::string target, config;          // custom_call
    std::vector<std::pair<std::vector<int64_t>, jh_dtype>> types;  // custom_call results
};

struct Program {
    size_t n_inputs = 0;
    int n_buffers = 0;
    std::vector<POp> ops;
};

const char* kTypeNames[] = {"f32", "f64", "f16", "bf16", "i1", "i8", "i32", "i64"};
bool is_type_name(const std::string& t) {
    for (const char* n : kTypeNames)
        if (t == n) return true;
    return false;
}

// "2x3xf32" -> {2, 3}: dimensions up to the first non-number (PJRT.cpp:517-537)
std::vector<int64_t> dims_of(const std::string& s, std::string* type = nullptr) {
    std::vector<int64_t> dims;
    std::istringstream ss(s);
    std::string tok;
    while (std::getline(ss, tok, 'x')) {
        if (is_type_name(tok)) {
            if (type) *type = tok;
            break;
        }
        char* end = nullptr;
        const long long v = std::strtoll(tok.c_str(), &end, 10);
        if (tok.empty() || end == tok.c_str()) {
            if (type) *type = tok;
            break;
        }
        dims.push_back(v);
    }
    return dims;
}

// floats separated by optional commas, read until the first failure
// (istringstream semantics of PJRT.cpp:472-477)
std::vector<float> floats_of(const std::string& s) {
    std::vector<float> v;
    std::istringstream ss(s);
    float x;
    while (ss >> x) {
        v.push_back(x);
        if (ss.peek() == ',') ss.ignore();
    }
    return v;
}
std::vector<int64_t> ints_of(const std::string& s) {
    std::vector<int64_t> v;
    std::istringstream ss(s);
    int64_t x;
    while (ss >> x) {
        v.push_back(x);
        if (ss.peek() == ',') ss.ignore();
    }
    return v;
}

std::vector<int64_t> parse_shape(const std::string& text, const std::string& name) {
    const std::regex rx("%" + name + "\\s*=\\s*\"[^\"]*\"\\([^)]*\\)[^{]*:\\s*tensor<([^>]+)>");
    for (auto it = std::sregex_iterator(text.begin(), text.end(), rx); it != std::sregex_iterator(); ++it) {
        auto d = dims_of((*it)[1].str());
        if (!d.empty()) return d;
    }
    return {};
}
std::vector<int64_t> parse_perm(const std::string& text, const std::string& name) {
    const std::regex rx("%" + name +
                        "\\s*=\\s*\"stablehlo\\.transpose\"\\([^)]*\\)\\s*\\{permutation\\s*=\\s*dense<\\[([^\\]]*)\\]>");
    for (auto it = std::sregex_iterator(text.begin(), text.end(), rx); it != std::sregex_iterator(); ++it) {
        auto p = ints_of((*it)[1].str());
        if (!p.empty()) return p;
    }
    return {};
}
std::vector<int64_t> parse_reduce_dims(const std::string& text, const std::string& name) {
    const std::regex op("%" + name + "\\s*=\\s*\"stablehlo\\.reduce\"[^}]*\\}");
    const std::regex dim("dimensions\\s*=\\s*dense<\\[([^\\]]*)\\]>");
    for (auto it = std::sregex_iterator(text.begin(), text.end(), op); it != std::sregex_iterator(); ++it) {
        const std::string t = (*it)[0].str();
        for (auto d = std::sregex_iterator(t.begin(), t.end(), dim); d != std::sregex_iterator(); ++d) {
            auto v = ints_of((*d)[1].str());
            if (!v.empty()) return v;
        }
    }
    return {};
}
std::vector<float> parse_const(const std::string& text, const std::string& name) {
    static const std::regex rx("%(\\w+)\\s*=\\s*\"stablehlo\\.constant\"\\(\\)\\s*\\{value\\s*=\\s*dense<([^>]*)>\\}");
    for (auto it = std::sregex_iterator(text.begin(), text.end(), rx); it != std::sregex_iterator(); ++it)
        if ((*it)[1].str() == name) return floats_of((*it)[2].str());
    return {};
}

// the rest of the op's line: custom_call attributes and result types
std::string line_from(const std::string& text, size_t pos) {
    const size_t e = text.find('\n', pos);
    return text.substr(pos, e == std::string::npos ? std::string::npos : e - pos);
}
std::string attr_string(const std::string& line, const char* key) {
    const std::regex rx(std::string(key) + "\\s*=\\s*\"([^\"]*)\"");
    std::smatch m;
    return std::regex_search(line, m, rx) ? m[1].str() : std::string();
}
jh_dtype dtype_of(const std::string& t) {
    if (t == "f32") return JH_F32;
    if (t == "bf16") return JH_BF16;
    if (t == "i8") return JH_I8;
    if (t == "i32") return JH_I32;
    fail(JH_ERR_DTYPE, "custom_call result type " + t + " (supported: f32, bf16, i8, i32)");
}

Program parse_program(const std::string& text, size_t n_inputs) {
    Program P;
    P.n_inputs = n_inputs;
    std::map<std::string, int> names;
    int next = 0;
    for (size_t i = 0; i < n_inputs; ++i) names["arg" + std::to_string(i)] = next++;
    auto ref = [&](const std::string& key) {
        auto it = names.find(key);
        if (it != names.end()) return it->second;
        names[key] = next;
        return next++;
    };
    static const std::regex op_rx("%(\\w+)(?::(\\d+))?\\s*=\\s*\"([\\w.]+)\"\\(([^)]*)\\)");
    static const std::regex operand_rx("%(\\w+)(?:#(\\d+))?");
    for (auto it = std::sregex_iterator(text.begin(), text.end(), op_rx); it != std::sregex_iterator(); ++it) {
        const std::smatch& m = *it;
        const std::string name = m[1].str(), opname = m[3].str(), operands = m[4].str();
        const int count = m[2].matched ? std::max(1, std::atoi(m[2].str().c_str())) : 1;
        POp op;
        op.opname = opname;
        for (auto o = std::sregex_iterator(operands.begin(), operands.end(), operand_rx); o != std::sregex_iterator(); ++o)
            op.ins.push_back(ref((*o)[2].matched ? (*o)[1].str() + "#" + (*o)[2].str() : (*o)[1].str()));
        for (int r = 0; r < count; ++r) {
            const int idx = next++;
            op.outs.push_back(idx);
            names[count == 1 ? name : name + "#" + std::to_string(r)] = idx;
        }
        if (count > 1) names[name] = op.outs[0];

        static const std::map<std::string, int> binary = {
            {"stablehlo.add", jh::PJ_ADD}, {"stablehlo.subtract", jh::PJ_SUB},
            {"stablehlo.multiply", jh::PJ_MUL}, {"stablehlo.divide", jh::PJ_DIV},
            {"stablehlo.maximum", jh::PJ_MAX}, {"stablehlo.minimum", jh::PJ_MIN}};
        static const std::map<std::string, int> unary = {
            {"stablehlo.negate", jh::PJ_NEG}, {"stablehlo.relu", jh::PJ_RELU},
            {"stablehlo.logistic", jh::PJ_SIGMOID}, {"stablehlo.tanh", jh::PJ_TANH},
            {"stablehlo.exponential", jh::PJ_EXP}, {"stablehlo.log", jh::PJ_LOG}};
        if (binary.count(opname)) {
            op.kind = POp::Binary;
            op.sub = binary.at(opname);
        } else if (unary.count(opname)) {
            op.kind = POp::Unary;
            op.sub = unary.at(opname);
        } else if (opname == "stablehlo.dot_general") {
            op.kind = POp::MatMul;
        } else if (opname == "stablehlo.reshape") {
            op.kind = POp::Reshape;
            op.shape = parse_shape(text, name);
        } else if (opname == "stablehlo.transpose") {
            op.kind = POp::Transpose;
            op.perm = parse_perm(text, name);
        } else if (opname == "stablehlo.reduce") {
            op.kind = POp::Reduce;
            op.dims = parse_reduce_dims(text, name);
        } else if (opname == "stablehlo.constant") {
            op.kind = POp::Constant;
            op.data = parse_const(text, name);
            if (op.data.empty()) op.data = {0.0f};
            op.shape = {(int64_t)op.data.size()};
        } else if (opname == "stablehlo.custom_call") {
            op.kind = POp::CustomCall;
            const std::string line = line_from(text, m.position(0) + m.length(0));
            op.target = attr_string(line, "call_target_name");
            op.config = attr_string(line, "backend_config");
            if (op.target.empty()) fail(JH_ERR_ARG, "custom_call %" + name + " has no call_target_name");
            const size_t arrow = line.rfind("->");
            if (arrow == std::string::npos)
                fail(JH_ERR_ARG, "custom_call %" + name + ": no result type after \"->\"");
            static const std::regex ty("tensor<([^>]*)>");
            const std::string res = line.substr(arrow);
            for (auto t = std::sregex_iterator(res.begin(), res.end(), ty); t != std::sregex_iterator(); ++t) {
                std::string tname = "f32";
                auto d = dims_of((*t)[1].str(), &tname);
                op.types.emplace_back(d, dtype_of(tname));
            }
            if ((int)op.types.size() != count)
                fail(JH_ERR_ARG, "custom_call %" + name + ": " + std::to_string(op.types.size()) +
                                     " result types for " + std::to_string(count) + " results");
        } else {
            op.kind = POp::Copy;  // unknown op: copy of operand 0 (or of buffer 0)
            if (op.ins.empty()) op.ins.push_back(0);
        }
        P.ops.push_back(std::move(op));
    }
    if (P.ops.empty()) {
        POp c;
        c.kind = POp::Copy;
        c.opname = "copy";
        c.ins = {0};
        c.outs = {next++};
        P.ops.push_back(c);
    }
    P.n_buffers = next;
    return P;
}

// ---------------------------------------------------------------------------
// Buffers and events
// ---------------------------------------------------------------------------
class ROCmBuffer : public DeviceBuffer {
public:
    ROCmBuffer(std::vector<int64_t> shape, jh_dtype t, int device, void* view = nullptr)
        : shape_(std::move(shape)), type_(t), device_(device), owned_(view == nullptr) {
        bytes_ = (size_t)elements(shape_) * dtype_size(t);
        if (view) {
            ptr_ = view;
        } else if (bytes_ > 0) {
            hip_check(hipSetDevice(device_), "hipSetDevice");
            hip_check(hipMalloc(&ptr_, bytes_), "hipMalloc");
        }
    }
    ~ROCmBuffer() override {
        if (owned_ && ptr_) {
            (void)hipSetDevice(device_);
            (void)hipFree(ptr_);
        }
    }
    size_t size() const override { return bytes_; }
    std::vector<int64_t> shape() const override { return shape_; }
    jh_dtype elementType() const override { return type_; }
    void copyFromHost(const void* data, size_t n) override {
        if (n > bytes_) fail(JH_ERR_SHAPE, "copyFromHost: more bytes than the buffer holds");
        hip_check(hipSetDevice(device_), "hipSetDevice");
        hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (n) hip_check(hipMemcpy(ptr_, data, n, hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    void copyToHost(void* data, size_t n) const override {
        if (n > bytes_) fail(JH_ERR_SHAPE, "copyToHost: more bytes than the buffer holds");
        hip_check(hipSetDevice(device_), "hipSetDevice");
        hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (n) hip_check(hipMemcpy(data, ptr_, n, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    }
    void* rawPointer() override { return ptr_; }
    int deviceId() const override { return device_; }
    bool isHostBuffer() const override { return false; }
    void setShape(std::vector<int64_t> s) { shape_ = std::move(s); }

private:
    std::vector<int64_t> shape_;
    jh_dtype type_;
    int device_;
    bool owned_;
    size_t bytes_ = 0;
    void* ptr_ = nullptr;
};

class ROCmEvent : public DeviceEvent {
public:
    ROCmEvent(int device, hipStream_t s) : device_(device) {
        hip_check(hipSetDevice(device), "hipSetDevice");
        hip_check(hipEventCreateWithFlags(&ev_, hipEventDisableTiming), "hipEventCreate");
        hip_check(hipEventRecord(ev_, s), "hipEventRecord");
    }
    ~ROCmEvent() override {
        (void)hipSetDevice(device_);
        (void)hipEventDestroy(ev_);
    }
    void await() override { hip_check(hipEventSynchronize(ev_), "hipEventSynchronize"); }
    bool isReady() const override { return hipEventQuery(ev_) == hipSuccess; }

private:
    int device_;
    hipEvent_t ev_ = nullptr;
};

// ---------------------------------------------------------------------------
// Executable
// ---------------------------------------------------------------------------
struct Val {
    std::shared_ptr<DeviceBuffer> buf;
    std::vector<int64_t> shape;
    bool present = false;
};

std::vector<int64_t> row_strides(const std::vector<int64_t>& shape) {
    std::vector<int64_t> s(shape.size(), 1);
    for (int i = (int)shape.size() - 2; i >= 0; --i) s[i] = s[i + 1] * shape[i + 1];
    return s;
}

class ROCmExecutable : public PJRTExecutable {
public:
    ROCmExecutable(std::string program, int device, hipStream_t stream)
        : program_(std::move(program)), device_(device), stream_(stream) {}

    std::vector<std::shared_ptr<DeviceBuffer>>
    execute(const std::vector<std::shared_ptr<DeviceBuffer>>& inputs) override {
        auto r = executeAsync(inputs);
        r.second->await();
        return r.first;
    }

    std::pair<std::vector<std::shared_ptr<DeviceBuffer>>, std::shared_ptr<DeviceEvent>>
    executeAsync(const std::vector<std::shared_ptr<DeviceBuffer>>& inputs) override {
        const Program& P = parsed(inputs.size());
        hip_check(hipSetDevice(device_), "hipSetDevice");
        std::vector<Val> v(P.n_buffers);
        for (size_t i = 0; i < inputs.size() && i < P.n_inputs; ++i) {
            if (!inputs[i]) fail(JH_ERR_NULL, "input " + std::to_string(i) + " is null");
            if (inputs[i]->deviceId() != device_ || inputs[i]->isHostBuffer())
                fail(JH_ERR_ARG, "input " + std::to_string(i) + " is not on device " + std::to_string(device_));
            v[i] = {inputs[i], inputs[i]->shape(), true};
        }
        for (const POp& op : P.ops) run(op, v);
        std::vector<std::shared_ptr<DeviceBuffer>> outs;
        for (int i = (int)P.n_inputs; i < P.n_buffers; ++i)
            if (v[i].present) outs.push_back(v[i].buf);
        if (outs.empty())
            for (const auto& in : inputs) {
                auto b = alloc(in->shape(), in->elementType());
                copy(b->rawPointer(), in->rawPointer(), in->size());
                outs.push_back(b);
            }
        return {outs, std::make_shared<ROCmEvent>(device_, stream_)};
    }

    std::string name() const override { return "rocm_executable"; }

    std::string describe(size_t n_inputs) {
        const Program& P = parsed(n_inputs);
        std::ostringstream os;
        static const char* kinds[] = {"binary", "unary", "matmul", "constant", "reshape",
                                      "transpose", "reduce", "custom_call", "copy"};
        auto list = [&](const std::vector<int64_t>& x) {
            std::string s = "[";
            for (size_t i = 0; i < x.size(); ++i) s += (i ? "," : "") + std::to_string(x[i]);
            return s + "]";
        };
        for (const POp& op : P.ops) {
            for (size_t i = 0; i < op.outs.size(); ++i) os << (i ? "," : "") << op.outs[i];
            os << " = " << kinds[op.kind] << " " << op.opname;
            for (int i : op.ins) os << " " << i;
            if (op.kind == POp::Binary || op.kind == POp::Unary) os << " sub=" << op.sub;
            if (op.kind == POp::Reshape) os << " shape=" << list(op.shape);
            if (op.kind == POp::Transpose) os << " perm=" << list(op.perm);
            if (op.kind == POp::Reduce) os << " dims=" << list(op.dims);
            if (op.kind == POp::Constant) {
                os << " data=[";
                for (size_t i = 0; i < op.data.size(); ++i) os << (i ? "," : "") << op.data[i];
                os << "]";
            }
            if (op.kind == POp::CustomCall) {
                os << " target=" << op.target << " config=\"" << op.config << "\" types=";
                for (auto& t : op.types) os << list(t.first) << ":" << (int)t.second << ";";
            }
            os << "\n";
        }
        os << "buffers " << P.n_buffers << "\n";
        return os.str();
    }

private:
    std::string program_;
    int device_;
    hipStream_t stream_;
    std::mutex mu_;
    std::map<size_t, Program> cache_;

    const Program& parsed(size_t n_inputs) {
        std::lock_guard<std::mutex> lock(mu_);
        auto it = cache_.find(n_inputs);
        if (it == cache_.end()) it = cache_.emplace(n_inputs, parse_program(program_, n_inputs)).first;
        return it->second;
    }

    std::shared_ptr<ROCmBuffer> alloc(const std::vector<int64_t>& shape, jh_dtype t) {
        return std::make_shared<ROCmBuffer>(shape, t, device_);
    }
    void copy(void* dst, const void* src, size_t bytes) {
        if (bytes) hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream_), "hipMemcpyAsync");
    }
    static const float* f32(const Val& x, const char* what) {
        if (x.buf->elementType() != JH_F32)
            fail(JH_ERR_DTYPE, std::string(what) + ": built-in ops take f32 buffers");
        return static_cast<const float*>(x.buf->rawPointer());
    }
    static int64_t count(const Val& x) { return (int64_t)(x.buf->size() / dtype_size(x.buf->elementType())); }
    void put(std::vector<Val>& v, int idx, std::shared_ptr<DeviceBuffer> b, std::vector<int64_t> shape) {
        v[idx] = {std::move(b), std::move(shape), true};
    }

    void run(const POp& op, std::vector<Val>& v) {
        auto have = [&](size_t k) { return k < op.ins.size() && v[op.ins[k]].present; };
        switch (op.kind) {
            case POp::Binary: {
                if (!have(0) || !have(1)) return;
                const Val &a = v[op.ins[0]], &b = v[op.ins[1]];
                const int64_t na = count(a), nb = count(b), n = std::max<int64_t>({na, nb, 1});
                // reference: the larger-rank operand's shape, the larger data size (:617-623)
                auto out = alloc({n}, JH_F32);
                hip_check(jh::launch_pj_binary(op.sub, f32(a, op.opname.c_str()), na, f32(b, op.opname.c_str()), nb,
                                               static_cast<float*>(out->rawPointer()), n, stream_),
                          op.opname.c_str());
                const auto& shape = a.shape.size() >= b.shape.size() ? a.shape : b.shape;
                out->setShape(elements(shape) == n ? shape : std::vector<int64_t>{n});
                put(v, op.outs[0], out, shape);
                return;
            }
            case POp::Unary: {
                if (!have(0)) return;
                const Val& a = v[op.ins[0]];
                const int64_t n = count(a);
                auto out = alloc({n}, JH_F32);
                hip_check(jh::launch_pj_unary(op.sub, f32(a, op.opname.c_str()),
                                              static_cast<float*>(out->rawPointer()), n, stream_),
                          op.opname.c_str());
                if (elements(a.shape) == n) out->setShape(a.shape);
                put(v, op.outs[0], out, a.shape);
                return;
            }
            case POp::Constant: {
                auto out = alloc(op.shape, JH_F32);
                hip_check(hipMemcpyAsync(out->rawPointer(), op.data.data(), op.data.size() * 4,
                                         hipMemcpyHostToDevice, stream_),
                          "constant upload");
                put(v, op.outs[0], out, op.shape);
                return;
            }
            case POp::MatMul: {
                if (!have(0) || !have(1)) return;
                const Val &a = v[op.ins[0]], &b = v[op.ins[1]];
                const auto& sa = a.shape;
                const auto& sb = b.shape;
                const int64_t M = sa.size() >= 2 ? sa[sa.size() - 2] : 1;
                const int64_t K = sa.size() >= 1 ? sa[sa.size() - 1] : 1;
                const int64_t N = sb.size() >= 2 ? sb[sb.size() - 1] : 1;
                if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
                    fail(JH_ERR_SHAPE, "dot_general: dimension above 2^31");
                if (count(a) < M * K || count(b) < K * N)
                    fail(JH_ERR_SHAPE, "dot_general: operand smaller than its M x K / K x N matrix");
                auto out = alloc({M, N}, JH_F32);
                if (M > 0 && N > 0)
                    hip_check(jh::launch_gemm_f32(JH_ACT_NONE, f32(a, "dot_general"), f32(b, "dot_general"),
                                                  nullptr, static_cast<float*>(out->rawPointer()), (int)M,
                                                  (int)N, (int)K, stream_),
                              "dot_general");
                put(v, op.outs[0], out, {M, N});
                return;
            }
            case POp::Reshape:
            case POp::Copy: {
                if (!have(0)) return;
                const Val& a = v[op.ins[0]];
                const std::vector<int64_t> shape =
                    (op.kind == POp::Reshape && !op.shape.empty()) ? op.shape : a.shape;
                auto out = alloc({count(a)}, a.buf->elementType());
                copy(out->rawPointer(), a.buf->rawPointer(), a.buf->size());
                if (elements(shape) == count(a)) out->setShape(shape);
                put(v, op.outs[0], out, shape);
                return;
            }
            case POp::Transpose: {
                if (!have(0)) return;
                const Val& a = v[op.ins[0]];
                const int rank = (int)a.shape.size();
                if (rank == 0) {
                    auto out = alloc({count(a)}, a.buf->elementType());
                    copy(out->rawPointer(), a.buf->rawPointer(), a.buf->size());
                    put(v, op.outs[0], out, a.shape);
                    return;
                }
                if (rank > 8) fail(JH_ERR_SHAPE, "transpose: rank above 8");
                std::vector<int64_t> perm = op.perm;
                if (perm.empty())
                    for (int d = rank - 1; d >= 0; --d) perm.push_back(d);
                std::vector<bool> seen(rank, false);
                if ((int)perm.size() != rank) fail(JH_ERR_ARG, "transpose: permutation length != rank");
                for (int64_t p : perm) {
                    if (p < 0 || p >= rank || seen[p]) fail(JH_ERR_ARG, "transpose: invalid permutation");
                    seen[p] = true;
                }
                const int64_t n = elements(a.shape);
                if (n != count(a)) fail(JH_ERR_SHAPE, "transpose: data size differs from its shape");
                std::vector<int64_t> out_shape(rank);
                for (int d = 0; d < rank; ++d) out_shape[d] = a.shape[perm[d]];
                const auto in_stride = row_strides(a.shape);
                jh::PjIndexMap map{};
                if (rank == 2) {  // the reference always swaps a rank-2 tensor (:768-777)
                    map.rank = 2;
                    map.out_stride[0] = a.shape[0];
                    map.out_stride[1] = 1;
                    map.in_step[0] = 1;
                    map.in_step[1] = a.shape[1];
                } else {
                    const auto os = row_strides(out_shape);
                    map.rank = rank;
                    for (int d = 0; d < rank; ++d) {
                        map.out_stride[d] = os[d];
                        map.in_step[d] = in_stride[perm[d]];
                    }
                }
                auto out = alloc(out_shape, JH_F32);
                hip_check(jh::launch_pj_transpose(f32(a, "transpose"), static_cast<float*>(out->rawPointer()),
                                                  n, map, stream_),
                          "transpose");
                put(v, op.outs[0], out, out_shape);
                return;
            }
            case POp::Reduce: {
                if (!have(0)) return;
                const Val& a = v[op.ins[0]];
                const int rank = (int)a.shape.size();
                if (rank == 0) {
                    auto out = alloc({count(a)}, a.buf->elementType());
                    copy(out->rawPointer(), a.buf->rawPointer(), a.buf->size());
                    put(v, op.outs[0], out, a.shape);
                    return;
                }
                if (rank > 8) fail(JH_ERR_SHAPE, "reduce: rank above 8");
                if (elements(a.shape) != count(a)) fail(JH_ERR_SHAPE, "reduce: data size differs from its shape");
                std::vector<bool> red(rank, op.dims.empty());
                for (int64_t d : op.dims)
                    if (d >= 0 && d < rank) red[d] = true;
                const auto in_stride = row_strides(a.shape);
                std::vector<int64_t> keep_shape, red_shape, keep_step, red_step;
                for (int d = 0; d < rank; ++d) {
                    (red[d] ? red_shape : keep_shape).push_back(a.shape[d]);
                    (red[d] ? red_step : keep_step).push_back(in_stride[d]);
                }
                std::vector<int64_t> out_shape = keep_shape.empty() ? std::vector<int64_t>{1} : keep_shape;
                jh::PjIndexMap keep{}, rmap{};
                keep.rank = (int)keep_shape.size();
                const auto ks = row_strides(keep_shape);
                for (int d = 0; d < keep.rank; ++d) {
                    keep.out_stride[d] = ks[d];
                    keep.in_step[d] = keep_step[d];
                }
                rmap.rank = (int)red_shape.size();
                const auto rs = row_strides(red_shape);
                for (int d = 0; d < rmap.rank; ++d) {
                    rmap.out_stride[d] = rs[d];
                    rmap.in_step[d] = red_step[d];
                }
                const int64_t n_out = elements(out_shape), n_red = elements(red_shape);
                auto out = alloc(out_shape, JH_F32);
                hip_check(jh::launch_pj_reduce(f32(a, "reduce"), static_cast<float*>(out->rawPointer()), n_out,
                                               n_red, keep, rmap, stream_),
                          "reduce");
                put(v, op.outs[0], out, out_shape);
                return;
            }
            case POp::CustomCall: {
                const std::string target = op.target == "gelu" ? "fusedGelu" : op.target;
                jh_kernel_fn fn = jules_hip_lookup(target.c_str());
                if (!fn) fail(JH_ERR_NOT_FOUND, "custom_call target \"" + op.target + "\" is not a registered kernel");
                std::vector<jh_tensor> ins(op.ins.size()), outs(op.types.size());
                std::vector<std::shared_ptr<ROCmBuffer>> out_bufs;
                auto desc = [](jh_tensor& t, void* data, const std::vector<int64_t>& shape, jh_dtype dt) {
                    if (shape.size() > 6) fail(JH_ERR_SHAPE, "custom_call: rank above 6");
                    std::memset(&t, 0, sizeof t);
                    t.data = data;
                    t.rank = (int32_t)shape.size();
                    t.dtype = dt;
                    const auto st = row_strides(shape);
                    for (size_t d = 0; d < shape.size(); ++d) {
                        t.sizes[d] = shape[d];
                        t.strides[d] = st[d];
                    }
                };
                for (size_t i = 0; i < op.ins.size(); ++i) {
                    const Val& a = v[op.ins[i]];
                    if (!a.present)
                        fail(JH_ERR_ARG, "custom_call " + op.target + ": operand " + std::to_string(i) + " has no value");
                    if (elements(a.shape) != count(a))
                        fail(JH_ERR_SHAPE, "custom_call " + op.target + ": operand " + std::to_string(i) +
                                               " data size differs from its shape");
                    desc(ins[i], a.buf->rawPointer(), a.shape, a.buf->elementType());
                }
                for (size_t r = 0; r < op.types.size(); ++r) {
                    out_bufs.push_back(alloc(op.types[r].first, op.types[r].second));
                    desc(outs[r], out_bufs.back()->rawPointer(), op.types[r].first, op.types[r].second);
                }
                const int st = fn((int)ins.size(), ins.data(), (int)outs.size(), outs.data(), op.config.c_str(),
                                  stream_);
                if (st != JH_OK)
                    fail(st, "custom_call " + op.target + ": " + jules_hip_last_error());
                for (size_t r = 0; r < op.types.size(); ++r) put(v, op.outs[r], out_bufs[r], op.types[r].first);
                return;
            }
        }
    }
};

// ---------------------------------------------------------------------------
// Device and client
// ---------------------------------------------------------------------------
class ROCmDevice : public PJRTDevice {
public:
    explicit ROCmDevice(int id) : id_(id) {
        hip_check(hipSetDevice(id), "hipSetDevice");
        hip_check(hipStreamCreate(&stream_), "hipStreamCreate");  // default priority
    }
    ~ROCmDevice() override {
        (void)hipSetDevice(id_);
        (void)hipStreamSynchronize(stream_);
        (void)hipStreamDestroy(stream_);
    }
    int id() const override { return id_; }
    std::string kind() const override { return "ROCM_GPU"; }
    std::string vendor() const override { return "AMD"; }
    size_t availableMemory() const override {
        size_t free_b = 0, total = 0;
        hip_check(hipSetDevice(id_), "hipSetDevice");
        hip_check(hipMemGetInfo(&free_b, &total), "hipMemGetInfo");
        return free_b;
    }
    std::shared_ptr<DeviceBuffer> allocateBuffer(const std::vector<int64_t>& shape, jh_dtype t) override {
        return std::make_shared<ROCmBuffer>(shape, t, id_);
    }
    std::shared_ptr<PJRTExecutable> loadExecutable(const std::string& program) override {
        return std::make_shared<ROCmExecutable>(program, id_, stream_);
    }
    hipStream_t stream() const { return stream_; }

private:
    int id_;
    hipStream_t stream_ = nullptr;
};

class ROCmClient : public PJRTClient {
public:
    ROCmClient() {
        int n = 0;
        hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
        if (n <= 0) fail(JH_ERR_HIP, "no ROCm device");
        for (int i = 0; i < n; ++i) devices_.push_back(std::make_unique<ROCmDevice>(i));
    }
    std::string platform() const override { return "rocm"; }
    size_t deviceCount() const override { return devices_.size(); }
    PJRTDevice* getDevice(size_t i) override { return i < devices_.size() ? devices_[i].get() : nullptr; }
    PJRTDevice* getDefaultDevice() override { return devices_[0].get(); }
    std::shared_ptr<DeviceBuffer> allocateBuffer(const std::vector<int64_t>& shape, jh_dtype t) override {
        return devices_[0]->allocateBuffer(shape, t);
    }
    std::shared_ptr<PJRTExecutable> compileAndLoad(const std::string& program) override {
        return devices_[0]->loadExecutable(program);
    }
    void synchronizeAll() override {
        for (auto& d : devices_) {
            hip_check(hipSetDevice(d->id()), "hipSetDevice");
            hip_check(hipStreamSynchronize(d->stream()), "hipStreamSynchronize");
        }
    }
    std::vector<std::shared_ptr<DeviceBuffer>>
    executePipeline(const std::vector<PJRTExecutable*>& stages,
                    const std::vector<std::shared_ptr<DeviceBuffer>>& inputs) override {
        if (stages.empty()) return {};
        std::vector<std::shared_ptr<DeviceBuffer>> cur = inputs;
        std::shared_ptr<DeviceEvent> last;
        for (PJRTExecutable* s : stages) {
            if (!s) fail(JH_ERR_NULL, "executePipeline: null stage");
            auto r = s->executeAsync(cur);  // same device stream: stream order chains the stages
            cur = std::move(r.first);
            last = std::move(r.second);
        }
        last->await();
        return cur;
    }

private:
    std::vector<std::unique_ptr<ROCmDevice>> devices_;
};

}  // namespace

std::unique_ptr<PJRTClient> PJRTClient::create(const std::string& platform) {
    if (platform != "rocm" && platform != "gpu")
        fail(JH_ERR_UNSUPPORTED, "platform \"" + platform + "\": this client serves \"rocm\"");
    return std::make_unique<ROCmClient>();
}

std::shared_ptr<DeviceBuffer> wrapDeviceMemory(void* data, const std::vector<int64_t>& shape,
                                               jh_dtype t, int device) {
    if (!data && elements(shape) > 0) fail(JH_ERR_NULL, "wrapDeviceMemory: null data");
    return std::make_shared<ROCmBuffer>(shape, t, device, data ? data : reinterpret_cast<void*>(16));
}

std::string describeProgram(const std::string& program, size_t n_inputs) {
    ROCmExecutable e(program, 0, nullptr);
    return e.describe(n_inputs);
}

}  // namespace jules_hip

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
struct jh_pjrt_exe {
    std::shared_ptr<jules_hip::PJRTClient> client;
    std::shared_ptr<jules_hip::PJRTExecutable> exe;
    std::vector<std::shared_ptr<jules_hip::DeviceBuffer>> last_outputs;
    int device = 0;
};

namespace {
template <typename F>
int guarded(F&& f) {
    try {
        return f();
    } catch (const jules_hip::PJRTError& e) {
        return jh::set_last_error(e.status(), e.what());
    } catch (const std::exception& e) {
        return jh::set_last_error(JH_ERR_ARG, e.what());
    } catch (...) {
        return jh::set_last_error(JH_ERR_ARG, "unknown error");
    }
}
}  // namespace

extern "C" {

int jules_hip_pjrt_describe(const char* program, int n_inputs, char* buf, size_t buf_len) {
    return guarded([&] {
        if (!program || !buf) return jh::set_last_error(JH_ERR_NULL, "pjrt_describe: null program or buffer");
        if (n_inputs < 0) return jh::set_last_error(JH_ERR_ARG, "pjrt_describe: negative input count");
        const std::string s = jules_hip::describeProgram(program, (size_t)n_inputs);
        if (s.size() + 1 > buf_len)
            return jh::set_last_error(JH_ERR_WORKSPACE, "pjrt_describe: buffer needs " + std::to_string(s.size() + 1) + " bytes");
        std::memcpy(buf, s.c_str(), s.size() + 1);
        return (int)JH_OK;
    });
}

int jules_hip_pjrt_compile(const char* program, int device, jh_pjrt_exe** out) {
    return guarded([&] {
        if (!program || !out) return jh::set_last_error(JH_ERR_NULL, "pjrt_compile: null program or out");
        *out = nullptr;
        auto client = std::shared_ptr<jules_hip::PJRTClient>(jules_hip::PJRTClient::create("rocm"));
        jules_hip::PJRTDevice* d = client->getDevice(device < 0 ? 0 : (size_t)device);
        if (!d) return jh::set_last_error(JH_ERR_ARG, "pjrt_compile: no device " + std::to_string(device));
        auto h = new jh_pjrt_exe;
        h->client = client;
        h->exe = d->loadExecutable(program);
        h->device = d->id();
        *out = h;
        return (int)JH_OK;
    });
}

int jules_hip_pjrt_execute(jh_pjrt_exe* h, int n_inputs, const jh_tensor* inputs, int max_outputs,
                           jh_tensor* outputs, int* n_outputs) {
    return guarded([&] {
        if (!h || (!inputs && n_inputs > 0) || !n_outputs || (!outputs && max_outputs > 0))
            return jh::set_last_error(JH_ERR_NULL, "pjrt_execute: null argument");
        if (n_inputs < 0 || max_outputs < 0) return jh::set_last_error(JH_ERR_ARG, "pjrt_execute: negative count");
        std::vector<std::shared_ptr<jules_hip::DeviceBuffer>> in;
        for (int i = 0; i < n_inputs; ++i) {
            const jh_tensor& t = inputs[i];
            if (t.rank < 0 || t.rank > 6) return jh::set_last_error(JH_ERR_SHAPE, "pjrt_execute: rank");
            std::vector<int64_t> shape(t.sizes, t.sizes + t.rank);
            int64_t expect = 1;
            for (int d = t.rank - 1; d >= 0; --d) {
                if (t.sizes[d] != 1 && t.strides[d] != expect)
                    return jh::set_last_error(JH_ERR_SHAPE, "pjrt_execute: inputs must be contiguous row-major");
                expect *= t.sizes[d];
            }
            char* base = static_cast<char*>(t.data) +
                         t.offset * (int64_t)(t.dtype == JH_BF16 ? 2 : t.dtype == JH_I8 ? 1 : 4);
            in.push_back(jules_hip::wrapDeviceMemory(base, shape, (jh_dtype)t.dtype, h->device));
        }
        h->last_outputs = h->exe->execute(in);
        *n_outputs = (int)h->last_outputs.size();
        if ((int)h->last_outputs.size() > max_outputs)
            return jh::set_last_error(JH_ERR_WORKSPACE, "pjrt_execute: " + std::to_string(h->last_outputs.size()) +
                                                            " outputs, room for " + std::to_string(max_outputs));
        for (size_t r = 0; r < h->last_outputs.size(); ++r) {
            auto& b = h->last_outputs[r];
            jh_tensor& t = outputs[r];
            std::memset(&t, 0, sizeof t);
            auto shape = b->shape();
            t.data = b->rawPointer();
            t.rank = (int32_t)std::min<size_t>(shape.size(), 6);
            t.dtype = b->elementType();
            int64_t st = 1;
            for (int d = t.rank - 1; d >= 0; --d) {
                t.sizes[d] = shape[d];
                t.strides[d] = st;
                st *= shape[d];
            }
        }
        return (int)JH_OK;
    });
}

int jules_hip_pjrt_destroy(jh_pjrt_exe* h) {
    return guarded([&] {
        delete h;
        return (int)JH_OK;
    });
}

}  // extern "C"
