// cPDE protocol server for one MI355X.
//
// Speaks the stdin/stdout frame protocol of the reference executable
// (cuda/protocol.hpp:10-51; opcodes cuda/cpde_server.cu:436-555) so that the
// reference's Python client and its cost, quadrature and checkpoint formats
// work unchanged against this executable.  All numerical work runs on the GPU
// through the device library's C ABI (include/cpde_hip.h); this file holds the
// object tables, request validation, the training loop, the scalar cost graph
// scheduling and the expression-cost code generation.
//
// Conventions of the reference that clients observe:
//   * a validation or numerical error answers kind 1 with a message and keeps
//     all server state (cuda/cpde_server.cu:22,573);
//   * a device failure prints to stderr and exits (cuda/cuda_check_v1.cuh:36-47);
//   * std::cout is redirected to stderr, stdout carries frames only;
//   * op 99 from the reader thread stops a running training between epochs.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <climits>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <iomanip>
#include <iostream>
#include <limits>
#include <map>
#include <memory>
#include <mutex>
#include <numeric>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "cpde_hip.h"

namespace {

// ---------------------------------------------------------------------------------------
// Errors: `Rejected` becomes a kind-1 reply, device failures end the process.
struct Rejected : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void require(bool ok, const char* message) {
    if (!ok) throw Rejected(message);
}

void call(int code) {
    if (code == CPDE_OK) return;
    const std::string message = cpde_last_error();
    if (code == CPDE_EINVAL || code == CPDE_ECOMPILE) throw Rejected(message);
    std::cerr << "cpde device failure: " << message << std::endl;
    std::exit(EXIT_FAILURE);
}

// ---------------------------------------------------------------------------------------
// Frames: uint64 LE length (counting the 4-byte kind), uint32 kind, payload.
// Arrays are uint64 count + raw elements, strings uint64 length + bytes.
struct Frame {
    std::vector<unsigned char> bytes;
    size_t pos = 0;

    template <class T>
    T get() {
        if (pos + sizeof(T) > bytes.size()) throw Rejected("truncated command");
        T v;
        std::memcpy(&v, bytes.data() + pos, sizeof v);
        pos += sizeof v;
        return v;
    }
    template <class T>
    std::vector<T> array() {
        const uint64_t n = get<uint64_t>();
        if (n > (bytes.size() - pos) / sizeof(T)) throw Rejected("truncated array");
        std::vector<T> v(n);
        if (n) std::memcpy(v.data(), bytes.data() + pos, n * sizeof(T));
        pos += n * sizeof(T);
        return v;
    }
    std::string string() {
        const auto a = array<char>();
        return std::string(a.begin(), a.end());
    }
    void end() const {
        if (pos != bytes.size()) throw Rejected("unexpected command fields");
    }
    bool more() const { return pos < bytes.size(); }

    template <class T>
    Frame& put(T v) {
        const auto* p = reinterpret_cast<const unsigned char*>(&v);
        bytes.insert(bytes.end(), p, p + sizeof v);
        return *this;
    }
    template <class T>
    Frame& put_array(const T* data, size_t n) {
        put<uint64_t>(n);
        const auto* p = reinterpret_cast<const unsigned char*>(data);
        bytes.insert(bytes.end(), p, p + n * sizeof(T));
        return *this;
    }
    template <class T>
    Frame& put_array(const std::vector<T>& v) {
        return put_array(v.data(), v.size());
    }
    Frame& put_string(const std::string& s) { return put_array(s.data(), s.size()); }
};

bool read_frame(Frame& f) {
    uint64_t n;
    if (std::fread(&n, 1, sizeof n, stdin) != sizeof n) return false;
    if (n < 4 || n > (uint64_t(4) << 30)) throw std::runtime_error("invalid frame size");
    f.bytes.resize(n);
    f.pos = 0;
    size_t got = 0;
    while (got < n) {
        const size_t k = std::fread(f.bytes.data() + got, 1, n - got, stdin);
        if (!k) throw std::runtime_error("truncated frame");
        got += k;
    }
    return true;
}

void send_frame(uint32_t kind, const Frame& f = Frame()) {
    const uint64_t n = 4 + f.bytes.size();
    if (std::fwrite(&n, 1, 8, stdout) != 8 || std::fwrite(&kind, 1, 4, stdout) != 4 ||
        (!f.bytes.empty() && std::fwrite(f.bytes.data(), 1, f.bytes.size(), stdout) != f.bytes.size()))
        throw std::runtime_error("response pipe closed");
    std::fflush(stdout);
}

int checked_size(int a, int b, int c = 1) {
    const int64_t n = int64_t(a) * b * c;
    require(a > 0 && b > 0 && c > 0 && n <= INT_MAX, "invalid or excessive dimensions");
    return int(n);
}

// ---------------------------------------------------------------------------------------
// Device memory owned by the server's records.
struct DeviceBuffer {
    cpde_device* dev = nullptr;
    void* ptr = nullptr;
    size_t bytes = 0;
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer() {
        if (ptr) cpde_buffer_free(dev, ptr);
    }
    void reset(cpde_device* d, size_t n) {
        if (ptr) call(cpde_buffer_free(dev, ptr));
        dev = d;
        ptr = nullptr;
        bytes = n;
        if (n) call(cpde_buffer_alloc(d, n, &ptr));
    }
    template <class T>
    void upload(cpde_device* d, const std::vector<T>& v) {
        reset(d, v.size() * sizeof(T));
        if (!v.empty()) call(cpde_buffer_upload(d, ptr, v.data(), bytes));
    }
    template <class T>
    T* as() const {
        return static_cast<T*>(ptr);
    }
};

// A derivative table: rows x (variables+1), row-major (order, counts...).
struct Table {
    int rows = 0, variables = 0;
    std::vector<int> cells;
    int order(int r) const { return cells[size_t(r) * (variables + 1)]; }
    int count(int r, int v) const { return cells[size_t(r) * (variables + 1) + 1 + v]; }
};

struct DataRecord {
    int rows = 0, channels = 0, samples = 0;  // d, h, w of op 2
    Table table;
    DeviceBuffer values;  // [row][sample][channel]
    uint64_t version = 0;
};

struct CostRecord;

struct NetRecord {
    cpde_net* net = nullptr;
    std::vector<int> neurons, linear;
    int optimizer = -1;
    uint64_t updates = 0, adam_step = 0, stage_done = 0, remaining = 0;
    float learning_rate = .001f, initial_step = .002f;
    std::string stage;
    // plans by (schema cells, width, backward); shared by costs with equal keys
    std::map<std::tuple<std::vector<int>, int, int>, cpde_plan*> plans;
    // the chunk currently in layer 0 (Server::activate, cuda/cpde_server.cu:158-170)
    struct Loaded {
        cpde_plan* plan = nullptr;
        uint64_t data = 0, version = 0, generation = 0;
        int offset = -1, valid = -1;
        std::vector<int> rows;
        bool operator==(const Loaded& o) const {
            return plan == o.plan && data == o.data && version == o.version && generation == o.generation &&
                   offset == o.offset && valid == o.valid && rows == o.rows;
        }
    } loaded;
    // the chunk in each plan's own input stack: re-activation is skipped while
    // it is unchanged, even when another plan's forward ran in between
    struct Input {
        uint64_t data = 0, version = 0;
        int offset = -1, valid = -1;
        std::vector<int> rows;
        bool operator==(const Input& o) const {
            return data == o.data && version == o.version && offset == o.offset && valid == o.valid && rows == o.rows;
        }
    };
    std::map<cpde_plan*, Input> inputs;
    // retained forward results: per cost, one stack set per chunk of its plan
    struct Retained {
        cpde_plan* plan = nullptr;
        std::vector<cpde_stacks*> sets;
    };
    std::map<uint64_t, Retained> retained;
    void drop_retained(uint64_t cost) {
        auto it = retained.find(cost);
        if (it == retained.end()) return;
        for (cpde_stacks* s : it->second.sets) cpde_stacks_destroy(s);
        retained.erase(it);
    }
    int transitions() const { return int(neurons.size()) - 1; }
    ~NetRecord() {
        for (auto& kv : retained)
            for (cpde_stacks* s : kv.second.sets) cpde_stacks_destroy(s);
        for (auto& kv : plans) cpde_plan_destroy(kv.second);
        if (net) cpde_net_destroy(net);
    }
};

struct ExpressionNode {
    int op, a, b;
    double parameter;
};

struct CostRecord {
    uint64_t net = 0, input = 0, target = 0;
    int kind = 0, width = 0;
    std::vector<int> rows;  // input-data rows forming the schema
    Table schema;
    DeviceBuffer row_map;   // rows, device (activation)
    // matching (kind 0)
    int weight_samples = 0;
    DeviceBuffer target_rows, weights;
    // polynomial (kind 1)
    int equations = 0, term_count = 0;
    DeviceBuffer terms, coefficients, rhs;
    // expression (kind 2)
    int samples = 0;
    std::vector<ExpressionNode> ir;
    std::string source;
    cpde_program* program = nullptr;  // owned by the server's program cache
    std::string log;
    DeviceBuffer fields, quadrature, scratch;
    bool has_components = true, has_gradient = true;
};

// ---------------------------------------------------------------------------------------
// Expression costs: per-sample double-precision forward of the IR and its
// reverse-mode adjoint, emitted as HIP source (the reference's generator is
// cuda/expression_program.hpp:20-66; semantics of the operators follow
// cuda/scalar_ops.cuh).  The generated kernel reads the output stack
// y[(point*rows + row)*outputs + output] (component index = row*outputs + output,
// row within the cost's schema).
enum Opcode { kConstant, kComponent, kField, kAdd, kSub, kMul, kDiv, kPower, kNeg, kExp, kLog, kSqrt, kSin, kCos, kTanh };

std::string number(double x) {
    std::ostringstream s;
    s << std::setprecision(17) << x;
    std::string t = s.str();
    if (t.find_first_of(".eEn") == std::string::npos) t += ".0";
    return t;
}

// The program of an expression cost (cuda/cost_kernels.cuh expression costs,
// cpde/_expressions.py IR): the gather of a sample's inputs from global memory
// (cpde_expression_inputs: its quadrature weight and the field values the
// program reads), a per-sample device function cpde_expression_point(yp, gp,
// inputs, ...) -- value, non-finite flag and, with `gradient`,
// d(loss)/d(output component) scaled by the multiplier into gp -- and the
// kernel `expression` that applies both to every sample of a chunk.  The
// library's one-pass epoch compiles the same functions into the network module,
// gathers a workgroup's inputs when it starts and applies the point function to
// the output values the workgroup holds in LDS.
std::string expression_source(const std::vector<ExpressionNode>& nodes) {
    std::ostringstream s;
    std::vector<int> field_ids;  // the fields the program reads, in order of first use
    std::map<int, int> field_slot;
    for (const ExpressionNode& n : nodes)
        if (n.op == kField && !field_slot.count(n.a)) {
            field_slot[n.a] = int(field_ids.size());
            field_ids.push_back(n.a);
        }
    s << "struct CpdeExpressionInputs {\n  double weight;\n  double field[" << std::max<size_t>(1, field_ids.size())
      << "];\n};\n"
         "// Sample p's inputs; one past `valid` reads the last valid sample's (not used).\n"
         "__device__ __forceinline__ CpdeExpressionInputs cpde_expression_inputs(const double* __restrict__ fields,\n"
         "    const double* __restrict__ weights, int samples, int offset, int p, int valid) {\n"
         "  CpdeExpressionInputs in{};\n"
         "  if (valid > 0) {\n"
         "    const int q = p < valid ? p : valid - 1;\n"
         "    in.weight = weights[offset + q];\n";
    for (size_t k = 0; k < field_ids.size(); ++k)
        s << "    in.field[" << k << "] = fields[" << field_ids[k] << " * (size_t)samples + offset + q];\n";
    s << "  }\n  return in;\n}\n"
         "__device__ __forceinline__ void cpde_expression_point(const float* __restrict__ yp, float* __restrict__ gp,\n"
         "    const CpdeExpressionInputs& in, int comps, int p, int valid, double scale, int collect, int gradient,\n"
         "    double* loss_out, int* bad_out) {\n"
         "  *loss_out = 0; *bad_out = -2;\n"
         "  if (gradient) for (int c = 0; c < comps; ++c) gp[c] = 0.0f;\n"
         "  if (p >= valid || in.weight == 0) return;\n"
         "  if (gradient && scale == 0 && !collect) return;\n"
         "  int bad = -2;\n"
         "  double lossv = 0;\n"
         "  {\n";
    std::vector<bool> active;
    for (size_t i = 0; i < nodes.size(); ++i) {
        const ExpressionNode& n = nodes[i];
        const std::string a = "v" + std::to_string(n.a), b = "v" + std::to_string(n.b);
        std::string e;
        switch (n.op) {
        case kConstant: e = number(n.parameter); break;
        case kComponent: e = "(double)yp[" + std::to_string(n.a) + "]"; break;
        case kField: e = "in.field[" + std::to_string(field_slot[n.a]) + "]"; break;
        case kAdd: e = a + " + " + b; break;
        case kSub: e = a + " - " + b; break;
        case kMul: e = a + " * " + b; break;
        case kDiv: e = "(" + b + " == 0 ? __builtin_nan(\"\") : " + a + " / " + b + ")"; break;
        case kPower:
            // a^1 and a^2 as a and a*a: pow's value there, with no call
            if (n.parameter == 1.0) e = a;
            else if (n.parameter == 2.0) e = a + " * " + a;
            else
                e = "((" + a + " < 0 && floor(" + number(n.parameter) + ") != " + number(n.parameter) + ") || (" + a +
                    " == 0 && " + number(n.parameter) + " < 0) ? __builtin_nan(\"\") : pow(" + a + ", " +
                    number(n.parameter) + "))";
            break;
        case kNeg: e = "-" + a; break;
        case kExp: e = "exp(" + a + ")"; break;
        case kLog: e = "(" + a + " > 0 ? log(" + a + ") : __builtin_nan(\"\"))"; break;
        case kSqrt: e = "(" + a + " >= 0 ? sqrt(" + a + ") : __builtin_nan(\"\"))"; break;
        case kSin: e = "sin(" + a + ")"; break;
        case kCos: e = "cos(" + a + ")"; break;
        case kTanh: e = "tanh(" + a + ")"; break;
        default: throw Rejected("invalid expression node");
        }
        s << "    const double v" << i << " = " << e << "; if (!isfinite(v" << i << ")) bad = -1;\n";
        const bool act = n.op == kComponent ? n.b == 0
                                            : (n.op <= kField ? false
                                                              : active[n.a] || (n.op >= kAdd && n.op <= kDiv && active[n.b]));
        active.push_back(act);
    }
    const size_t last = nodes.size() - 1;
    s << "    if (collect) lossv = in.weight * v" << last << ";\n"
      << "    if (!isfinite(lossv)) bad = -1;\n"
      << "    *loss_out = lossv; *bad_out = bad;\n"
      << "    if (!gradient || scale == 0 || bad != -2) return;\n";
    for (size_t i = 0; i < nodes.size(); ++i) s << "    double d" << i << " = " << (i == last ? "1" : "0") << ";\n";
    for (int i = int(nodes.size()) - 1; i >= 0; --i) {
        const ExpressionNode& n = nodes[i];
        if (n.op <= kField || !active[i]) continue;
        const std::string a = "v" + std::to_string(n.a), b = "v" + std::to_string(n.b), v = "v" + std::to_string(i);
        std::string da = "0", db = "0";
        switch (n.op) {
        case kAdd: da = db = "1"; break;
        case kSub: da = "1"; db = "-1"; break;
        case kMul: da = b; db = a; break;
        case kDiv: da = "1 / " + b; db = "-" + v + " / " + b; break;
        case kPower:
            da = n.parameter == 0 ? "0"
                                  : (n.parameter == 1 ? "1"
                                                      : (n.parameter == 2 ? "2.0 * " + a
                                                                          : number(n.parameter) + " * pow(" + a + ", " +
                                                                                number(n.parameter - 1) + ")"));
            break;
        case kNeg: da = "-1"; break;
        case kExp: da = v; break;
        case kLog: da = "1 / " + a; break;
        case kSqrt: da = "0.5 / " + v; break;
        case kSin: da = "cos(" + a + ")"; break;
        case kCos: da = "-sin(" + a + ")"; break;
        case kTanh: da = "1 - " + v + " * " + v; break;
        }
        s << "    if (d" << i << " != 0) {";
        if (active[n.a]) s << " d" << n.a << " += d" << i << " * (" << da << ");";
        if (n.op >= kAdd && n.op <= kDiv && active[n.b]) s << " d" << n.b << " += d" << i << " * (" << db << ");";
        s << " }\n";
    }
    // repeated components are summed in double before the fp32 store
    std::map<int, std::vector<size_t>> comps;
    for (size_t i = 0; i < nodes.size(); ++i)
        if (nodes[i].op == kComponent && nodes[i].b == 0) comps[nodes[i].a].push_back(i);
    for (const auto& kv : comps) {
        s << "    { double t = 0";
        for (size_t i : kv.second) s << " + d" << i;
        s << "; const float out = (float)(t * in.weight * scale); gp[" << kv.first
          << "] = out; if (!isfinite(out)) *bad_out = " << kv.first << "; }\n";
    }
    s << "  }\n}\n"
         "extern \"C\" __global__ __launch_bounds__(256) void expression(const float* __restrict__ y, float* g,\n"
         "    const double* __restrict__ fields, const double* __restrict__ weights, double* loss, int* bad,\n"
         "    int outputs, int rows, int samples, int width, int offset, int valid, const double* multiplier,\n"
         "    int collect, int gradient) {\n"
         "  const int comps = rows * outputs;\n"
         "  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < width; p += blockDim.x * gridDim.x) {\n"
         "    const double scale = multiplier ? *multiplier : 1.0;\n"
         "    const CpdeExpressionInputs in = cpde_expression_inputs(fields, weights, samples, offset, p, valid);\n"
         "    cpde_expression_point(y + (size_t)p * comps, gradient ? g + (size_t)p * comps : nullptr, in, comps, p,\n"
         "                          valid, scale, collect, gradient, &loss[p], &bad[p]);\n"
         "  }\n}\n";
    return s.str();
}

// ---------------------------------------------------------------------------------------
// Scalar cost graph (cuda/cost_graph.cuh, cuda/graph_schedule.hpp): leaves are
// cost values, the root the training objective.  Before any cost is evaluated
// the schedule decides which leaf multipliers d(root)/d(leaf) are already known
// (constants and linear structure); those leaves run forward and backward in
// one pass, the others after the graph has been evaluated.
enum GraphOp { gConstant = 0, gLeaf = 1, gAdd = 3, gSub, gMul, gDiv, gPower, gNeg, gExp, gLog, gSqrt, gSin, gCos, gTanh, gAttach };

double scalar_value(int op, double a, double b, double p) {
    switch (op) {
    case gConstant: return p;
    case gAdd: return a + b;
    case gSub: return a - b;
    case gMul: return a * b;
    case gDiv: return b == 0 ? NAN : a / b;
    case gPower: return ((a < 0 && std::floor(p) != p) || (a == 0 && p < 0)) ? NAN : std::pow(a, p);
    case gNeg: return -a;
    case gExp: return std::exp(a);
    case gLog: return a > 0 ? std::log(a) : NAN;
    case gSqrt: return a >= 0 ? std::sqrt(a) : NAN;
    case gSin: return std::sin(a);
    case gCos: return std::cos(a);
    case gTanh: return std::tanh(a);
    case gAttach: return a;
    default: return NAN;
    }
}

void scalar_partials(int op, double a, double b, double v, double p, double& da, double& db) {
    da = db = 0;
    switch (op) {
    case gAdd:
    case gAttach: da = db = 1; break;
    case gSub: da = 1; db = -1; break;
    case gMul: da = b; db = a; break;
    case gDiv: da = 1 / b; db = -v / b; break;
    case gPower: da = p == 0 ? 0 : (p == 1 ? 1 : p * std::pow(a, p - 1)); break;
    case gNeg: da = -1; break;
    case gExp: da = v; break;
    case gLog: da = 1 / a; break;
    case gSqrt: da = .5 / v; break;
    case gSin: da = std::cos(a); break;
    case gCos: da = -std::sin(a); break;
    case gTanh: da = 1 - v * v; break;
    default: break;
    }
}

struct Known {
    bool known;
    double value;
};
Known known(double v) { return {std::isfinite(v), v}; }
Known add_known(Known a, Known b) { return a.known && b.known ? known(a.value + b.value) : Known{false, 0}; }
Known mul_known(Known a, Known b) {
    if ((a.known && a.value == 0) || (b.known && b.value == 0)) return known(0);
    return a.known && b.known ? known(a.value * b.value) : Known{false, 0};
}

// Which leaf multipliers are fixed before evaluation (dependency analysis only).
std::vector<Known> schedule_leaves(const std::vector<cpde_scalar_node>& nodes, int root, int leaves) {
    const Known unknown{false, 0};
    const size_t N = nodes.size();
    std::vector<Known> value(N, unknown), da(N, unknown), db(N, unknown);
    std::vector<bool> active(N, false);
    for (size_t i = 0; i < N; ++i) {
        const auto& n = nodes[i];
        if (n.op == gConstant) {
            value[i] = known(n.parameter);
            continue;
        }
        if (n.op == gLeaf) {
            active[i] = true;
            continue;
        }
        const bool binary = n.op <= gDiv || n.op == gAttach;
        const Known a = value[n.a], b = binary ? value[n.b] : known(0);
        active[i] = active[n.a] || (binary && active[n.b]);
        if (a.known && (b.known || n.op == gAttach)) value[i] = known(scalar_value(n.op, a.value, b.value, n.parameter));
        if (n.op == gAdd || n.op == gAttach) da[i] = db[i] = known(1);
        else if (n.op == gSub) {
            da[i] = known(1);
            db[i] = known(-1);
        } else if (n.op == gMul) {
            da[i] = b;
            db[i] = a;
        } else if (n.op == gDiv) {
            if (b.known && b.value != 0) {
                da[i] = known(1 / b.value);
                if (a.known) db[i] = known(-(a.value / b.value) / b.value);
            }
        } else if (n.op == gNeg)
            da[i] = known(-1);
        else if (n.op == gPower && (n.parameter == 0 || n.parameter == 1))
            da[i] = known(n.parameter);
        else if (a.known && value[i].known) {
            double x, y;
            scalar_partials(n.op, a.value, b.value, value[i].value, n.parameter, x, y);
            da[i] = known(x);
        }
    }
    std::vector<Known> adjoint(N, known(0)), multipliers(leaves, known(0));
    adjoint[root] = known(1);
    for (int i = int(N) - 1; i >= 0; --i) {
        const auto& n = nodes[i];
        const Known seed = adjoint[i];
        if (!active[i] || (seed.known && seed.value == 0)) continue;
        if (n.op == gLeaf) multipliers[n.a] = add_known(multipliers[n.a], seed);
        else {
            if (active[n.a]) adjoint[n.a] = add_known(adjoint[n.a], mul_known(seed, da[i]));
            if ((n.op <= gDiv || n.op == gAttach) && active[n.b]) adjoint[n.b] = add_known(adjoint[n.b], mul_known(seed, db[i]));
        }
    }
    return multipliers;
}

struct GraphRecord {
    std::vector<cpde_scalar_node> nodes;
    int root = 0, leaves = 0;
    std::vector<Known> schedule;
    // the summary is written into the device's own slot (cpde_graph_execute with
    // a null summary) and arrives with the scalar download
    DeviceBuffer dev_nodes, values, adjoints, multipliers, active, fixed;
    cpde_graph_summary host{0, -1, 0};

    void read(cpde_device* dev, Frame& b, int leaf_count) {
        const auto raw = b.array<int>();
        const auto constants = b.array<double>();
        root = b.get<int>();
        require(!constants.empty() && constants.size() <= 4096 && raw.size() == 3 * constants.size() && root >= 0 &&
                    root < int(constants.size()),
                "invalid cost graph size");
        leaves = leaf_count;
        for (int i = 0; i < int(constants.size()); ++i) {
            const int op = raw[3 * i], a = raw[3 * i + 1], c = raw[3 * i + 2];
            require(std::isfinite(constants[i]), "nonfinite graph constant");
            require(op == gConstant || op == gLeaf || (op >= gAdd && op <= gAttach), "invalid graph opcode");
            if (op == gLeaf) require(a >= 0 && a < leaves, "invalid graph leaf");
            if (op >= gAdd) {
                require(a >= 0 && a < i, "graph must be topologically ordered");
                if (op <= gDiv || op == gAttach) require(c >= 0 && c < i, "invalid graph child");
            }
            nodes.push_back(cpde_scalar_node{op, a, c, 0, constants[i]});
        }
        dev_nodes.upload(dev, nodes);
        values.reset(dev, nodes.size() * sizeof(double));
        adjoints.reset(dev, nodes.size() * sizeof(double));
        active.reset(dev, nodes.size() * sizeof(int));
        multipliers.reset(dev, std::max(1, leaves) * sizeof(double));
        schedule = schedule_leaves(nodes, root, leaves);
        std::vector<double> f(std::max(1, leaves), 0.0);
        for (int i = 0; i < leaves; ++i)
            if (schedule[i].known) f[i] = schedule[i].value;
        fixed.upload(dev, f);
    }
    void validate() const {
        if (host.bad_node >= 0)
            throw Rejected(("invalid value or derivative in cost graph node " + std::to_string(host.bad_node)).c_str());
    }
};

// ---------------------------------------------------------------------------------------
class Server {
public:
    // The device is opened by the first command that needs it, so the
    // handshake and request validation work on a machine without a GPU.
    explicit Server(int ordinal) : ordinal_(ordinal) {}
    ~Server() {
        if (dev_ && !trace_file_.empty()) write_trace();
        if (const char* path = std::getenv("CPDE_REPLAY_FILE")) {
            if (std::FILE* f = std::fopen(path, "w")) {
                std::fprintf(f, "{\"recorded\": %llu, \"replayed\": %llu, \"ahead\": %llu}\n",
                             (unsigned long long)recorded_, (unsigned long long)replayed_,
                             (unsigned long long)ahead_);
                std::fclose(f);
            }
        }
        costs_.clear();
        nets_.clear();
        data_.clear();
        for (auto& kv : programs_) cpde_program_destroy(kv.second);
        if (dev_) cpde_device_close(dev_);
    }

    void command(uint32_t op, Frame& b, std::atomic<bool>& stop);

private:
    int ordinal_ = 0;
    cpde_device* dev_ = nullptr;
    uint64_t next_id_ = 1;
    // With CPDE_TRACE_FILE set, every launch of the session is timed per kernel
    // class and the totals are written there as JSON when the server ends.
    std::string trace_file_;
    static double retain_budget_mb() {
        const char* v = std::getenv("CPDE_RETAIN_MB");
        return v && *v ? std::max(0.0, std::atof(v)) : 16384.0;
    }
    void open_device() {
        if (dev_) return;
        call(cpde_device_open(ordinal_, &dev_));
        if (const char* path = std::getenv("CPDE_TRACE_FILE")) {
            trace_file_ = path;
            call(cpde_trace_enable(dev_, 1));
        }
    }
    void write_trace() {
        std::FILE* f = std::fopen(trace_file_.c_str(), "w");
        if (!f) return;
        std::fprintf(f, "{");
        bool first = true;
        for (int k = 0; k < cpde_trace_kinds(); ++k) {
            uint64_t launches = 0;
            double ms = 0, work = 0;
            if (cpde_trace_read(dev_, k, &launches, &ms, &work) != CPDE_OK || launches == 0) continue;
            std::fprintf(f, "%s\"%s\": [%llu, %.9g, %.17g]", first ? "" : ", ", cpde_trace_name(k),
                         (unsigned long long)launches, ms, work);
            first = false;
        }
        std::fprintf(f, "}\n");
        std::fclose(f);
    }
    std::unordered_map<uint64_t, std::unique_ptr<DataRecord>> data_;
    std::unordered_map<uint64_t, std::unique_ptr<NetRecord>> nets_;
    std::unordered_map<uint64_t, std::unique_ptr<CostRecord>> costs_;
    std::unordered_map<std::string, cpde_program*> programs_;
    int cost_slots_ = 0;

    template <class M>
    static typename M::mapped_type::element_type& lookup(M& m, uint64_t id) {
        auto it = m.find(id);
        require(it != m.end(), "unknown or released object handle");
        return *it->second;
    }
    DataRecord& data(uint64_t id) { return lookup(data_, id); }
    NetRecord& net(uint64_t id) { return lookup(nets_, id); }
    CostRecord& cost(uint64_t id) { return lookup(costs_, id); }

    // rows of `d` sorted by order, stable (Server::all_rows, cuda/cpde_server.cu:124-127)
    static std::vector<int> all_rows(const DataRecord& d) {
        std::vector<int> rows(d.rows);
        std::iota(rows.begin(), rows.end(), 0);
        std::stable_sort(rows.begin(), rows.end(), [&](int a, int b) { return d.table.order(a) < d.table.order(b); });
        return rows;
    }

    // schema from selected data rows (Server::make_schema, cuda/cpde_server.cu:113-123)
    static Table make_schema(const DataRecord& d, const std::vector<int>& rows) {
        require(!rows.empty(), "empty derivative closure");
        Table s;
        s.rows = int(rows.size());
        s.variables = d.table.variables;
        int previous = -1;
        for (int src : rows) {
            require(src >= 0 && src < d.rows, "invalid derivative row");
            const int order = d.table.order(src);
            require(order >= previous && order <= 6, "derivative closure must be sorted, orders 0..6");
            previous = order;
            for (int c = 0; c <= d.table.variables; ++c) s.cells.push_back(d.table.cells[size_t(src) * (s.variables + 1) + c]);
        }
        require(s.cells[0] == 0, "value derivative must come first");
        return s;
    }

    cpde_plan* plan_for(NetRecord& n, const Table& schema, int width, bool backward) {
        const auto key = std::make_tuple(schema.cells, width, backward ? 1 : 0);
        auto it = n.plans.find(key);
        if (it != n.plans.end()) return it->second;
        cpde_plan* p = nullptr;
        call(cpde_plan_create(n.net, schema.rows, schema.variables, schema.cells.data(), width, backward ? 1 : 0, &p));
        n.plans.emplace(key, p);
        return p;
    }

    void reserve_slots(int costs) {
        if (costs > cost_slots_) {
            call(cpde_costs_begin(dev_, costs));
            cost_slots_ = costs;
        }
    }

    // Server::activate (cuda/cpde_server.cu:158-170): copy a chunk into layer 0,
    // skipped when that chunk is already there.
    void activate(NetRecord& n, cpde_plan* plan, uint64_t data_id, const std::vector<int>& rows, int offset, int valid);

    struct Pass {
        bool backward, collect;
        const double* multiplier;
        int begin, end;
        bool reuse_forward;
        // 1: each chunk's forward goes into the cost's retained stack set for
        // that chunk; 2: the cost and backward run on the retained forward
        // (`id` names the cost)
        int retain = 0;
        uint64_t id = 0;
    };
    bool retention_fits(NetRecord& n, CostRecord& c, double& budget);
    static double stack_set_bytes(const NetRecord& n, const CostRecord& c);
    double retained_elsewhere(NetRecord& n, const std::vector<uint64_t>& ids);
    void bind_retained(NetRecord& n, uint64_t id, cpde_plan* plan, int chunk);
    void pass(NetRecord& n, CostRecord& c, int slot, bool& first, const Pass& how);
    void prepare_costs(NetRecord& n, const std::vector<uint64_t>& ids, uint64_t ni);
    void graph_pass(NetRecord& n, const std::vector<uint64_t>& ids, GraphRecord& graph, bool backward,
                    bool leave_waiting = false);
    bool retained_last_ = false;  // the last graph pass kept forwards in stack sets

    // An epoch's backward passes over one network share their reduction
    // launches (cpde_gradients_defer: two passes per launch, the graph riding
    // in it); CPDE_DEFER_REDUCE=0 reduces every pass in its own launch.
    struct DeferredReductions {
        cpde_device* dev = nullptr;
        DeferredReductions(cpde_device* d, bool on) {
            const char* v = std::getenv("CPDE_DEFER_REDUCE");
            if (on && !(v && *v && std::atoi(v) == 0)) {
                call(cpde_gradients_defer(d, 1));
                dev = d;
            }
        }
        void finish() {
            if (dev) call(cpde_gradients_defer(dev, 0));
            dev = nullptr;
        }
        // the waiting launches stay waiting for the caller, who ends deferral
        void release() { dev = nullptr; }
        ~DeferredReductions() {
            if (dev) (void)cpde_gradients_defer(dev, 0);
        }
    };
    // epochs recorded and replayed, and first halves sent ahead of the previous
    // epoch's checks (written to CPDE_REPLAY_FILE when the server ends)
    uint64_t recorded_ = 0, replayed_ = 0, ahead_ = 0;

    // Captured epochs (CPDE_REPLAY=1): from the second epoch of a training call
    // on, an epoch's gradient work (its passes, the graph and the gradient
    // statistics) is recorded once per (active-buffer parity, collect) with
    // cpde_capture_begin and replayed as one HIP graph launch; the scalar
    // download, the validation and the optimizer update stay separate host
    // calls, as in the reference's loop.  Off by default: on ROCm 7.2 a
    // replayed epoch took longer than the same launches issued one by one
    // (Poisson disk graph epoch 0.103 ms against 0.092-0.097; a three-launch
    // matching epoch about 5 us more, with or without a synchronisation per
    // epoch).
    struct EpochReplays {
        bool on = false;
        int refusals = 0;
        std::map<std::pair<int, int>, cpde_replay*> cache;
        ~EpochReplays() { clear(); }
        void clear() {
            for (auto& kv : cache) (void)cpde_replay_destroy(kv.second);
            cache.clear();
        }
    };
    static bool replay_enabled() {
        const char* v = std::getenv("CPDE_REPLAY");
        return v && *v && std::atoi(v) != 0;
    }
    void gradient_epoch(EpochReplays& r, NetRecord& n, bool warm, bool collect, const std::function<void()>& work);
    void download_rprop(NetRecord& n, int costs, int layers, std::vector<cpde_cost_stats>& cs,
                        std::vector<cpde_gradient_stats>& gs, GraphRecord* graph, int& updated);
    // A training epoch in two halves: its passes up to the deferred gradient
    // launches, then the graph, those launches and the gradient statistics.
    bool halves_apply(const std::vector<uint64_t>& ids, const GraphRecord* graph);
    void first_half(NetRecord& n, const std::vector<uint64_t>& ids, GraphRecord* graph, bool collect);
    void second_half(NetRecord& n, int costs, int layers, bool graph, int method, bool full_stats);
    void download(int costs, int layers, std::vector<cpde_cost_stats>& cs, std::vector<cpde_gradient_stats>& gs,
                  GraphRecord* graph = nullptr);
    void validate_costs(const std::vector<cpde_cost_stats>& cs, std::vector<double>& values, bool before_update);
    void evaluate_costs(NetRecord& n, const std::vector<uint64_t>& ids, std::vector<double>& values, GraphRecord* graph);
    uint64_t evaluate(uint64_t ni, uint64_t di, int chunk);
    void reset_optimizer(NetRecord& n, int method);
    Frame metadata(const NetRecord& n) const;
    Frame snapshot(NetRecord& n);
    void restore(NetRecord& n, Frame& b);
    void train(Frame& b, std::atomic<bool>& stop, bool graph_mode);
    void timing(Frame& b, Frame& out);
    uint64_t create_cost(Frame& b);
    uint64_t create_integral(Frame& b);
};


// ---------------------------------------------------------------------------------------
void Server::activate(NetRecord& n, cpde_plan* plan, uint64_t data_id, const std::vector<int>& rows, int offset,
                      int valid) {
    DataRecord& d = data(data_id);
    NetRecord::Loaded want{plan, data_id, d.version, cpde_net_generation(n.net), offset, valid, rows};
    if (n.loaded == want) return;
    const NetRecord::Input in{data_id, d.version, offset, valid, rows};
    auto it = n.inputs.find(plan);
    if (it == n.inputs.end() || !(it->second == in)) {
        call(cpde_activate(plan, d.values.as<float>(), d.samples, rows.data(), offset, valid));
        n.inputs[plan] = in;
    }
    want.generation = cpde_net_generation(n.net);
    n.loaded = want;
}

// One cost over its chunks (Server::pass, cuda/cpde_server.cu:223-257): forward,
// the cost with its reduction into `slot`, and (backward) the adjoint pass with
// the first backward of an epoch overwriting the gradient.
void Server::pass(NetRecord& n, CostRecord& c, int slot, bool& first, const Pass& how) {
    if (!c.input) return;
    const bool backward = how.backward && c.has_gradient;
    DataRecord& input = data(c.input);
    const int end = std::min(how.end, input.samples);
    require(how.begin >= 0 && how.begin % c.width == 0 && (!how.reuse_forward || int64_t(end) - how.begin <= c.width),
            "invalid cost pass range");
    cpde_plan* plan = plan_for(n, c.schema, c.width, true);
    for (int offset = how.begin; offset < end; offset += c.width) {
        const int valid = std::min(c.width, input.samples - offset);
        if (how.retain) {
            bind_retained(n, how.id, plan, offset / c.width);
            if (how.retain == 1) {  // this chunk's forward, kept in its own stack set
                call(cpde_activate(plan, input.values.as<float>(), input.samples, c.rows.data(), offset, valid));
                if (c.has_components) call(cpde_forward(plan));
            }
        } else if (how.reuse_forward) {
            DataRecord& d = data(c.input);
            const NetRecord::Loaded want{plan, c.input, d.version, cpde_net_generation(n.net), offset, valid, c.rows};
            require(n.loaded == want, "forward context is no longer current");
        } else {
            activate(n, plan, c.input, c.rows, offset, valid);
            if (c.kind == 2 && backward && c.has_components) {
                // forward, cost and backward of this chunk in one pass (the
                // multiplier, if any, is final before the pass starts)
                call(cpde_epoch_expression(plan, c.program, c.fields.as<double>(), c.quadrature.as<double>(), c.samples,
                                           offset, valid, how.multiplier, c.scratch.ptr, slot, how.collect,
                                           first ? 0 : 1));
                first = false;
                continue;
            }
            if (c.kind == 0 && backward && !how.multiplier && c.has_components) {
                // forward, cost and backward of this chunk in one pass
                DataRecord& t = data(c.target);
                call(cpde_epoch_matching(plan, t.values.as<float>(), t.samples, c.target_rows.as<int>(),
                                         c.weights.as<float>(), c.weight_samples, offset, valid, slot, how.collect,
                                         first ? 0 : 1));
                first = false;
                continue;
            }
            if (c.has_components) call(cpde_forward(plan));
        }
        if (c.kind == 0) {
            DataRecord& t = data(c.target);
            call(cpde_cost_matching(plan, t.values.as<float>(), t.samples, c.target_rows.as<int>(), c.weights.as<float>(),
                                    c.weight_samples, offset, valid, slot, how.collect, backward));
        } else if (c.kind == 1) {
            call(cpde_cost_polynomial(plan, c.terms.as<cpde_poly_term>(), c.term_count, c.coefficients.as<float>(),
                                      c.rhs.as<float>(), c.weights.as<float>(), c.equations, input.samples, offset, valid,
                                      slot, how.collect, backward));
        } else {
            call(cpde_cost_expression(plan, c.program, c.fields.as<double>(), c.quadrature.as<double>(), c.samples, offset,
                                      valid, how.multiplier, c.scratch.ptr, slot, how.collect, backward));
        }
        if (backward && how.multiplier && c.kind != 2) call(cpde_scale_adjoint(plan, how.multiplier));
        if (backward) {
            call(cpde_backward(plan, first ? 0 : 1));
            first = false;
        }
        if (how.retain) call(cpde_plan_bind(plan, nullptr));
    }
}

// Retention of forward results (the reference's plan, IMPLEMENTATION_PLAN.md:750-831;
// its engine recomputes instead, cuda/cpde_server.cu:273-318): a cost whose
// multiplier depends on the graph's values keeps every chunk's forward in a
// stack set of its own between the value pass and the backward, while the sets
// of all such costs fit CPDE_RETAIN_MB (default 16384; 0: recompute, as the
// reference does).  `budget` is what is left of it.  An expression cost whose
// backward runs as one launch with the forward inside it keeps its forwards
// only when a chunk's forward is large (2^28 multiply-adds and up): below that
// the separate cost and backward launches cost more than the recomputation.
// Measured per epoch of a two-leaf graph whose value-dependent leaf has one
// row: 2->128^3->1 on 2048-point chunks (6.8e7 multiply-adds) 0.478 ms kept,
// 0.455 recomputed; 2->256^3->1 on 4096-point chunks (5.4e8) 0.574 kept,
// 0.597 recomputed; 2->512^3->1 (no one-launch backward) 5.64 kept, 6.68
// recomputed.
bool Server::retention_fits(NetRecord& n, CostRecord& c, double& budget) {
    if (!c.input || !c.has_gradient || !c.has_components) return false;
    const int samples = data(c.input).samples;
    const double chunks = std::ceil(double(samples) / c.width);
    const double columns = double(c.width) * c.schema.rows;
    if (c.kind == 2) {
        int fused = 0;
        call(cpde_epoch_expression_fused(plan_for(n, c.schema, c.width, true), c.program, &fused));
        double macs = 0;
        for (size_t l = 0; l + 1 < n.neurons.size(); ++l) macs += double(n.neurons[l]) * n.neurons[l + 1];
        if (fused && macs * columns < std::ldexp(1.0, 28)) return false;
    }
    const double bytes = chunks * stack_set_bytes(n, c);
    if (bytes > budget) return false;
    budget -= bytes;
    return true;
}

// One chunk's stack set: per layer y, and z or u where the layer composes,
// and g past the input layer; plus the chunk's input.
double Server::stack_set_bytes(const NetRecord& n, const CostRecord& c) {
    const double columns = double(c.width) * c.schema.rows;
    double floats = columns * n.neurons[0];
    for (size_t l = 0; l < n.neurons.size(); ++l)
        floats += columns * n.neurons[l] * (1 + (n.linear[l] ? 0 : 1) + (l > 0 ? 1 : 0));
    return floats * sizeof(float);
}

// Bytes of stack sets the network holds for costs outside `ids`: they stay
// allocated through this pass, so they come off the retention budget.
double Server::retained_elsewhere(NetRecord& n, const std::vector<uint64_t>& ids) {
    double bytes = 0;
    for (const auto& kv : n.retained) {
        if (std::find(ids.begin(), ids.end(), kv.first) != ids.end()) continue;
        auto it = costs_.find(kv.first);
        if (it == costs_.end()) continue;
        bytes += double(kv.second.sets.size()) * stack_set_bytes(n, *it->second);
    }
    return bytes;
}

void Server::bind_retained(NetRecord& n, uint64_t id, cpde_plan* plan, int chunk) {
    auto& r = n.retained[id];
    if (r.plan != plan) {  // a new plan for this cost (chunk width or schema changed)
        for (cpde_stacks* set : r.sets) cpde_stacks_destroy(set);
        r.sets.clear();
        r.plan = plan;
    }
    while (int(r.sets.size()) <= chunk) {
        cpde_stacks* set = nullptr;
        call(cpde_stacks_create(plan, &set));
        r.sets.push_back(set);
    }
    call(cpde_plan_bind(plan, r.sets[chunk]));
}

// Server::prepare_costs (cuda/cpde_server.cu:258-272): costs belong to this net,
// programs compiled, plans and reduction slots in place.
void Server::prepare_costs(NetRecord& n, const std::vector<uint64_t>& ids, uint64_t ni) {
    for (uint64_t id : ids) {
        CostRecord& c = cost(id);
        require(c.net == ni, "cost belongs to another network");
        if (c.kind == 2 && !c.program) {
            auto it = programs_.find(c.source);
            if (it == programs_.end()) {
                cpde_program* prog = nullptr;
                std::vector<char> log(1 << 16);
                const int code = cpde_program_compile(dev_, c.source.c_str(), &prog, log.data(), log.size());
                c.log = log.data();
                call(code);
                it = programs_.emplace(c.source, prog).first;
            }
            c.program = it->second;
        }
        if (c.input) plan_for(n, c.schema, c.width, true);
    }
    reserve_slots(int(ids.size()));
}

// Cost and gradient scalars, and the graph summary of the last graph pass, in
// one synchronisation (Workspace::download, cuda/reduction_kernels.cuh:171-177).
void Server::download(int costs, int layers, std::vector<cpde_cost_stats>& cs, std::vector<cpde_gradient_stats>& gs,
                      GraphRecord* graph) {
    cs.resize(std::max(costs, 1));
    gs.resize(std::max(layers, 1));
    if (graph)
        call(cpde_scalars_download_graph(dev_, costs, cs.data(), layers, gs.data(),
                                         nullptr, &graph->host));
    else
        call(cpde_scalars_download(dev_, costs, cs.data(), layers, gs.data()));
    cs.resize(costs);
    gs.resize(layers);
}

// download(), with the network's RPROP update launched behind the copy; it
// applies only if the epoch passes the checks that train() makes next.
void Server::download_rprop(NetRecord& n, int costs, int layers, std::vector<cpde_cost_stats>& cs,
                            std::vector<cpde_gradient_stats>& gs, GraphRecord* graph, int& updated) {
    cs.resize(std::max(costs, 1));
    gs.resize(std::max(layers, 1));
    call(cpde_scalars_download_rprop(dev_, costs, cs.data(), layers, gs.data(), graph ? &graph->host : nullptr, n.net,
                                     &updated));
    cs.resize(costs);
    gs.resize(layers);
}

// Whether train() may run its epochs in halves and send the next
// epoch's first half before this epoch's scalars are back
// (CPDE_EPOCH_HALVES=0: never).  The first half writes stacks, cost records,
// partials and the graph's values and multipliers, all scratch, while its
// last gradient launches wait.  Reductions it must launch early (the graph
// riding in one, a third pass, a cost slot finished twice) store into the
// gradient buffers only if the update issued before them applied: the
// update's kernel leaves its verdict on the device and those reductions read
// it.  So a rejected epoch drops the next one's first half and keeps every
// state buffer as whole epochs keep it.  That needs deferred reductions and,
// with a graph, a leaf that writes the gradient (a graph pass with none
// zeroes it instead, unconditionally).
bool Server::halves_apply(const std::vector<uint64_t>& ids, const GraphRecord* graph) {
    const char* v = std::getenv("CPDE_EPOCH_HALVES");
    const char* d = std::getenv("CPDE_DEFER_REDUCE");
    if ((v && *v && std::atoi(v) == 0) || (d && *d && std::atoi(d) == 0) || ids.size() > 64) return false;
    if (!graph) return true;
    for (size_t i = 0; i < ids.size(); ++i) {  // graph_pass's test for a leaf that writes the gradient
        CostRecord& c = cost(ids[i]);
        const bool runs = !graph->schedule[i].known || graph->schedule[i].value != 0;
        if (runs && c.input && c.has_gradient && data(c.input).samples > 0) return true;
    }
    return false;
}

// The first half: the graph pass (the graph itself included) or the plain
// cost list's passes, their gradient launches left waiting.
void Server::first_half(NetRecord& n, const std::vector<uint64_t>& ids, GraphRecord* graph, bool collect) {
    if (graph) {
        graph_pass(n, ids, *graph, true, true);
        return;
    }
    call(cpde_costs_begin(dev_, int(ids.size())));
    call(cpde_gradients_defer(dev_, 1));
    bool first = true;
    for (size_t i = 0; i < ids.size(); ++i)
        pass(n, cost(ids[i]), int(i), first, Pass{true, collect, nullptr, 0, INT_MAX, false});
}

// The second half: the waiting gradient launches, then the statistics and
// the update issued in one call (the update applies only if the epoch passes
// the checks, which cpde_update_resolve reports).  full_stats: the whole
// gradient statistics are reported this epoch; otherwise the library may hand
// out short ones, and a rejected epoch's are taken whole afterwards.
void Server::second_half(NetRecord& n, int costs, int layers, bool graph, int method, bool full_stats) {
    call(cpde_gradients_defer(dev_, 0));
    call(cpde_inspect_update_issue(dev_, costs, layers, graph ? 1 : 0, n.net, method,
                                   method == 1 ? int(n.adam_step + 1) : 0, n.learning_rate, full_stats ? 1 : 0));
}

// Server::validate_costs (cuda/cpde_server.cu:341-352).
void Server::validate_costs(const std::vector<cpde_cost_stats>& cs, std::vector<double>& values, bool before_update) {
    const std::string phase =
        before_update ? "; no optimizer update performed for this iteration" : " during objective evaluation";
    for (size_t i = 0; i < cs.size(); ++i) {
        values[i] = cs[i].value;
        if (cs[i].bad_sample != INT_MAX) {
            const std::string what = cs[i].bad_component < 0 ? std::string("objective")
                                                             : "dE/dY component " + std::to_string(cs[i].bad_component);
            throw Rejected(("non-finite " + what + " at cost index " + std::to_string(i) + ", sample " +
                            std::to_string(cs[i].bad_sample) + phase)
                               .c_str());
        }
        if (!std::isfinite(cs[i].value)) throw Rejected(("non-finite reduced objective" + phase).c_str());
    }
}

// Server::graph_pass (cuda/cpde_server.cu:273-318).  `leave_waiting`: the
// deferred gradient launches (with the graph riding in the reduction, where it
// does) are left waiting for the caller.
void Server::graph_pass(NetRecord& n, const std::vector<uint64_t>& ids, GraphRecord& graph, bool backward,
                        bool leave_waiting) {
    call(cpde_costs_begin(dev_, int(ids.size())));
    DeferredReductions deferred(dev_, backward);
    bool first = true;
    int reuse = -1, last_offset = 0;
    double best_work = -1;
    std::vector<char> keep(ids.size(), 0);  // leaves whose forwards are retained until their backward
    retained_last_ = false;
    if (backward) {
        // The reference zeroes the gradient here (cuda/cpde_server.cu:278).  The
        // first backward pass overwrites all of it (accumulate 0), so the zero
        // fill is needed only when no leaf will run one.
        bool written = false;
        for (size_t i = 0; i < ids.size() && !written; ++i) {
            CostRecord& c = cost(ids[i]);
            const bool runs = !graph.schedule[i].known || graph.schedule[i].value != 0;
            written = runs && c.input && c.has_gradient && data(c.input).samples > 0;
        }
        if (!written) call(cpde_zero_gradient(n.net));
        double budget = retain_budget_mb() * 1048576.0 - retained_elsewhere(n, ids);
        for (size_t i = 0; i < ids.size(); ++i)
            if (!graph.schedule[i].known && retention_fits(n, cost(ids[i]), budget)) keep[i] = retained_last_ = true;
        // run the most expensive leaf with an unknown multiplier and no
        // retained forwards last, so its final forward can be reused by its
        // backward (a work estimate)
        for (size_t i = 0; i < ids.size(); ++i) {
            if (graph.schedule[i].known || keep[i]) continue;
            CostRecord& c = cost(ids[i]);
            if (!c.input || !c.has_gradient || !c.has_components) continue;
            double derivative_work = 0, work = 0;
            for (int r = 0; r < c.schema.rows; ++r) derivative_work += std::ldexp(1.0, c.schema.order(r));
            for (size_t l = 0; l + 1 < n.neurons.size(); ++l) {
                work += 2.0 * n.neurons[l] * n.neurons[l + 1] * c.rows.size();
                if (n.linear[l] == 0) work += n.neurons[l] * derivative_work;
            }
            work *= c.width;
            if (work > best_work) {
                best_work = work;
                reuse = int(i);
            }
        }
    }
    const double* fixed = graph.fixed.as<double>();
    const double* multipliers = graph.multipliers.as<double>();
    for (size_t i = 0; i < ids.size(); ++i) {
        if (int(i) == reuse) continue;
        const bool immediate = backward && graph.schedule[i].known && graph.schedule[i].value != 0;
        pass(n, cost(ids[i]), int(i), first,
             Pass{immediate, true, immediate ? fixed + i : nullptr, 0, INT_MAX, false, keep[i] ? 1 : 0, ids[i]});
    }
    if (reuse >= 0) {
        CostRecord& c = cost(ids[reuse]);
        last_offset = ((data(c.input).samples - 1) / c.width) * c.width;
        pass(n, c, reuse, first, Pass{false, true, nullptr, 0, INT_MAX, false});
    }
    call(cpde_graph_execute(dev_, graph.dev_nodes.as<cpde_scalar_node>(), int(graph.nodes.size()), graph.root,
                            int(ids.size()), graph.values.as<double>(), graph.adjoints.as<double>(),
                            graph.multipliers.as<double>(), graph.active.as<int>(),
                            nullptr, backward ? 1 : 0));
    if (backward) {
        if (reuse >= 0)
            pass(n, cost(ids[reuse]), reuse, first,
                 Pass{true, false, multipliers + reuse, last_offset, INT_MAX, true});
        for (size_t i = 0; i < ids.size(); ++i)
            if (!graph.schedule[i].known)
                pass(n, cost(ids[i]), int(i), first,
                     Pass{true, false, multipliers + i, 0, int(i) == reuse ? last_offset : INT_MAX, false,
                          keep[i] ? 2 : 0, ids[i]});
    }
    if (leave_waiting) deferred.release();
    else deferred.finish();
}

void Server::evaluate_costs(NetRecord& n, const std::vector<uint64_t>& ids, std::vector<double>& values,
                            GraphRecord* graph) {
    std::vector<cpde_cost_stats> cs;
    std::vector<cpde_gradient_stats> gs;
    if (graph) {
        graph_pass(n, ids, *graph, false);
        download(int(ids.size()), 0, cs, gs, graph);
        validate_costs(cs, values, false);
        graph->validate();
        return;
    }
    call(cpde_costs_begin(dev_, int(ids.size())));
    bool unused = true;
    for (size_t i = 0; i < ids.size(); ++i)
        pass(n, cost(ids[i]), int(i), unused, Pass{false, true, nullptr, 0, INT_MAX, false});
    download(int(ids.size()), 0, cs, gs);
    validate_costs(cs, values, false);
}

// Server::evaluate (cuda/cpde_server.cu:171-183): forward every row of `di`
// chunk by chunk into a new data object [row][sample][output].
uint64_t Server::evaluate(uint64_t ni, uint64_t di, int chunk) {
    NetRecord& n = net(ni);
    DataRecord& input = data(di);
    require(input.channels == n.neurons.front(), "input channel mismatch");
    const int width = chunk ? std::min(chunk, input.samples) : input.samples;
    require(width > 0, "invalid chunk size");
    const std::vector<int> rows = all_rows(input);
    const Table schema = make_schema(input, rows);
    cpde_plan* plan = plan_for(n, schema, width, false);
    auto out = std::make_unique<DataRecord>();
    out->rows = input.rows;
    out->channels = n.neurons.back();
    out->samples = input.samples;
    out->table = input.table;
    out->values.reset(dev_, size_t(input.rows) * input.samples * out->channels * sizeof(float));
    for (int offset = 0; offset < input.samples; offset += width) {
        const int valid = std::min(width, input.samples - offset);
        activate(n, plan, di, rows, offset, valid);
        call(cpde_forward(plan));
        call(cpde_output(plan, out->values.as<float>(), out->samples, rows.data(), offset, valid));
    }
    call(cpde_device_synchronize(dev_));
    const uint64_t id = next_id_++;
    data_[id] = std::move(out);
    return id;
}

// Server::reset (cuda/cpde_server.cu:184-192).
void Server::reset_optimizer(NetRecord& n, int method) {
    call(cpde_reset_optimizer(n.net));
    if (method == 0) call(cpde_set_steps(n.net, n.initial_step));
    n.optimizer = method;
    n.adam_step = 0;
}

// Snapshot blob (cuda/cpde_server.cu:193-206).
Frame Server::metadata(const NetRecord& n) const {
    Frame b;
    b.put<uint32_t>(1).put_array(n.neurons).put_array(n.linear).put<int32_t>(n.optimizer);
    b.put<uint64_t>(n.updates).put<uint64_t>(n.adam_step).put<uint64_t>(n.stage_done).put<uint64_t>(n.remaining);
    b.put<float>(n.learning_rate).put<float>(n.initial_step).put_string(n.stage);
    return b;
}

Frame Server::snapshot(NetRecord& n) {
    call(cpde_device_synchronize(dev_));
    Frame b = metadata(n);
    for (int t = 0; t < n.transitions(); ++t) {
        b.put<int32_t>(cpde_net_active(n.net, t));
        for (int k = 0; k < 4; ++k) {
            float* ptr = nullptr;
            int count = 0;
            call(cpde_net_state(n.net, t, k, &ptr, &count));
            std::vector<float> v(count);
            call(cpde_buffer_download(dev_, v.data(), ptr, v.size() * sizeof(float)));
            b.put_array(v);
        }
    }
    return b;
}

void Server::restore(NetRecord& n, Frame& b) {
    require(b.get<uint32_t>() == 1, "unsupported state version");
    require(b.array<int>() == n.neurons && b.array<int>() == n.linear, "state architecture mismatch");
    const int optimizer = b.get<int32_t>();
    require(optimizer >= -1 && optimizer <= 1, "invalid optimizer state");
    const uint64_t updates = b.get<uint64_t>(), adam = b.get<uint64_t>(), done = b.get<uint64_t>(),
                   remaining = b.get<uint64_t>();
    const float lr = b.get<float>(), step = b.get<float>();
    const std::string stage = b.string();
    require(std::isfinite(lr) && lr > 0 && std::isfinite(step) && step > 0, "invalid optimizer settings");
    std::vector<int> active;
    std::vector<std::vector<float>> arrays;
    for (int t = 0; t < n.transitions(); ++t) {
        const int a = b.get<int32_t>();
        require(a == 1 || a == 2, "invalid active gradient buffer");
        active.push_back(a);
        const size_t count = size_t(n.neurons[t + 1]) * (n.neurons[t] + 1);
        for (int k = 0; k < 4; ++k) {
            arrays.push_back(b.array<float>());
            require(arrays.back().size() == count, "state buffer shape mismatch");
        }
    }
    b.end();
    call(cpde_device_synchronize(dev_));
    for (int t = 0; t < n.transitions(); ++t) {
        call(cpde_net_set_active(n.net, t, active[t]));
        for (int k = 0; k < 4; ++k) {
            float* ptr = nullptr;
            int count = 0;
            call(cpde_net_state(n.net, t, k, &ptr, &count));
            const auto& v = arrays[size_t(t) * 4 + k];
            call(cpde_buffer_upload(dev_, ptr, v.data(), v.size() * sizeof(float)));
        }
    }
    n.optimizer = optimizer;
    n.updates = updates;
    n.adam_step = adam;
    n.stage_done = done;
    n.remaining = remaining;
    n.learning_rate = lr;
    n.initial_step = step;
    n.stage = stage;
}

// One epoch's gradient work: replayed when a recording of it exists for the
// network's current active gradient buffers, recorded when none does (the
// recording runs once as it ends), otherwise issued launch by launch.  A
// replay that the library refuses (memory released or state moved since the
// capture) drops every recording of the call; after three refusals, or when a
// recording cannot be made, the call issues its epochs launch by launch.
void Server::gradient_epoch(EpochReplays& r, NetRecord& n, bool warm, bool collect,
                            const std::function<void()>& work) {
    if (!r.on || !warm) return work();
    const std::pair<int, int> key{cpde_net_active(n.net, 0), collect ? 1 : 0};
    auto it = r.cache.find(key);
    if (it != r.cache.end()) {
        if (cpde_replay_launch(it->second) == CPDE_OK) {
            ++replayed_;
            return;
        }
        r.clear();
        if (++r.refusals > 2) r.on = false;
    }
    // stack sets bound per chunk, or a device that is tracing launches: no recording
    if (!r.on || retained_last_) {
        r.on = false;
        return work();
    }
    if (cpde_capture_begin(dev_) != CPDE_OK) {
        std::cerr << "cpde_server: epochs not recorded: " << cpde_last_error() << std::endl;
        r.on = false;
        return work();
    }
    bool recorded = true;
    try {
        work();
    } catch (const std::exception& e) {
        std::cerr << "cpde_server: epoch not recorded: " << e.what() << std::endl;
        recorded = false;
    }
    cpde_replay* made = nullptr;
    if (recorded) {
        if (cpde_capture_end(dev_, 1, &made) == CPDE_OK && made) {
            r.cache[key] = made;
            ++recorded_;
            return;
        }
        std::cerr << "cpde_server: epoch not recorded: " << cpde_last_error() << std::endl;
    } else {
        (void)cpde_capture_end(dev_, 0, nullptr);
    }
    // nothing that was recorded ran: the chunks it activated are not in place
    n.loaded = NetRecord::Loaded{};
    n.inputs.clear();
    r.on = false;
    work();
}

// Server::train (cuda/cpde_server.cu:364-435): the epoch loop with validation
// before every optimizer step, event frames and the final metadata reply.
void Server::train(Frame& b, std::atomic<bool>& stop, bool graph_mode) {
    const uint64_t ni = b.get<uint64_t>();
    NetRecord& n = net(ni);
    const auto ids = b.array<uint64_t>();
    const uint64_t epochs = b.get<uint64_t>();
    const int method = b.get<int32_t>(), fresh = b.get<int32_t>();
    const float steps = b.get<float>();
    const int moments = b.get<int32_t>();
    const float lr = b.get<float>();
    const int verbose = b.get<int32_t>(), log = b.get<int32_t>(), eval = b.get<int32_t>(), outputs = b.get<int32_t>(),
              save = b.get<int32_t>();
    (void)verbose;
    const std::string stage = b.string();
    const int diagnostics = b.get<int32_t>();
    std::unique_ptr<GraphRecord> graph;
    if (graph_mode) {
        graph = std::make_unique<GraphRecord>();
        graph->read(dev_, b, int(ids.size()));
    }
    uint64_t restore_every = 0;
    float restore_step = 0;
    if (b.more()) {
        restore_every = b.get<uint64_t>();
        restore_step = b.get<float>();
    }
    b.end();
    require(!ids.empty() && epochs > 0, "training needs costs and positive epochs");
    require(method == 0 || method == 1, "unknown optimizer");
    require(ids.size() <= INT_MAX && log >= 0 && eval >= 0 && save >= 0 && diagnostics >= 0 && std::isfinite(lr) &&
                lr >= 0 && std::isfinite(steps) && steps >= 0,
            "invalid training controls");
    require((restore_every == 0 && restore_step == 0) ||
                (restore_every > 0 && method == 0 && std::isfinite(restore_step) &&
                 restore_step >= std::numeric_limits<float>::min()),
            "invalid periodic RPROP restoration controls");
    prepare_costs(n, ids, ni);
    if (fresh || n.optimizer != method) reset_optimizer(n, method);
    if (lr > 0) n.learning_rate = lr;
    if (steps > 0) {
        require(method == 0, "reset_steps requires RPROP");
        call(cpde_set_steps(n.net, steps));
    }
    if (moments) {
        require(method == 1, "reset_moments requires Adam");
        reset_optimizer(n, 1);
    }
    if (graph) {
        if (n.stage.substr(0, n.stage.find('|')) != stage.substr(0, stage.find('|'))) n.stage_done = 0;
        n.stage = stage;
    } else if (n.stage != stage) {
        n.stage = stage;
        n.stage_done = 0;
    }
    n.remaining = epochs;
    const int layers = n.transitions();
    std::vector<double> values(ids.size());
    std::vector<cpde_cost_stats> cs;
    std::vector<cpde_gradient_stats> gs;
    uint64_t completed = 0, last_saved = UINT64_MAX, last_eval = UINT64_MAX;
    auto report = [&](int after) {
        Frame r;
        r.put<uint64_t>(completed).put<uint64_t>(n.updates).put<int32_t>(after).put_array(values);
        if (graph) r.put<double>(graph->host.value);
        send_frame(graph ? 6 : 2, r);
    };
    EpochReplays replays;
    replays.on = replay_enabled() && epochs >= 4;
    // Epochs in halves: the next epoch's first half goes out behind this
    // epoch's update, before its scalars are back, unless the host acts on the
    // device between the two (evaluation, snapshot, step restoration, the
    // end); a stop request then takes effect one update later.  If the checks
    // reject this epoch, the next one's first half is dropped.
    const bool halves = !replays.on && halves_apply(ids, graph.get());
    bool ahead = false;  // the next epoch's first half is out
    // leaving early: a first half sent ahead is dropped, waiting launches of
    // this epoch's go out (deferral ends, as DeferredReductions ends it)
    struct Ahead {
        cpde_device* dev;
        bool& on;
        bool used;
        ~Ahead() {
            if (!used) return;
            if (on) (void)cpde_gradients_discard(dev);
            else (void)cpde_gradients_defer(dev, 0);
        }
    } ahead_guard{dev_, ahead, halves};
    auto collect_at = [&](uint64_t done) { return (log && (done + 1) % log == 0) || done + 1 == epochs; };
    // the epochs after which the gradient statistics are reported (event 5)
    auto reports_diagnostics = [&](uint64_t done) {
        return diagnostics && ((done + 1) % diagnostics == 0 || done + 1 == epochs);
    };
    while (completed < epochs && (ahead || !stop.load())) {
        const bool collect = collect_at(completed);
        // RPROP goes out behind the download and applies only if the checks
        // below pass (the library applies the same rule to the same scalars)
        const bool fused_update = method == 0 && ids.size() <= 64;
        int updated = 0;
        if (halves) {
            if (!ahead) first_half(n, ids, graph.get(), collect);
            ahead = false;
            require(method == 0 || n.adam_step < uint64_t(INT_MAX), "Adam counter exceeds supported range");
            const bool full_stats = reports_diagnostics(completed);
            second_half(n, int(ids.size()), layers, graph != nullptr, method, full_stats);
            const uint64_t next = completed + 1;
            const bool acts = next == epochs || (eval && next % eval == 0) || (save && next % save == 0) ||
                              (restore_every && (n.updates + 1) % restore_every == 0) || stop.load();
            if (!acts) {
                ahead = true;
                try {
                    first_half(n, ids, graph.get(), collect_at(next));
                    ++ahead_;
                } catch (...) {
                    // dropped; the next iteration sends it whole, after this
                    // epoch is counted, where whole epochs would have failed
                    (void)cpde_gradients_discard(dev_);
                    ahead = false;
                }
            }
            cs.resize(std::max<size_t>(ids.size(), 1));
            gs.resize(std::max(layers, 1));
            call(cpde_update_resolve(dev_, cs.data(), gs.data(), graph ? &graph->host : nullptr, &updated));
            cs.resize(ids.size());
            gs.resize(layers);
            bool short_bad = false;
            for (const auto& g : gs) short_bad = short_bad || (!full_stats && g.nonfinite_count != 0);
            if (short_bad) {
                // the report of a rejected epoch: its untouched gradients' whole
                // statistics, after the next epoch's first half is dropped (the
                // statistics launch would send its waiting launches out, no
                // longer gated on the resolved update)
                if (ahead) {
                    call(cpde_gradients_discard(dev_));
                    ahead = false;
                }
                call(cpde_inspect_gradients(n.net));
                call(cpde_scalars_download(dev_, 0, nullptr, layers, gs.data()));
            }
        } else {
            gradient_epoch(replays, n, completed > 0, collect, [&] {
                if (graph) graph_pass(n, ids, *graph, true);
                else {
                    call(cpde_costs_begin(dev_, int(ids.size())));
                    DeferredReductions deferred(dev_, true);
                    bool first = true;
                    for (size_t i = 0; i < ids.size(); ++i)
                        pass(n, cost(ids[i]), int(i), first, Pass{true, collect, nullptr, 0, INT_MAX, false});
                    deferred.finish();
                }
                call(cpde_inspect_gradients(n.net));
            });
            if (fused_update) download_rprop(n, int(ids.size()), layers, cs, gs, graph.get(), updated);
            else download(int(ids.size()), layers, cs, gs, graph.get());
        }
        bool bad_gradient = false;
        for (const auto& g : gs) bad_gradient = bad_gradient || g.nonfinite_count != 0;
        if (bad_gradient || reports_diagnostics(completed)) {
            Frame r;
            r.put<uint64_t>(completed + 1).put<uint64_t>(n.updates).put<int32_t>(layers);
            for (const auto& g : gs)
                r.put<double>(g.squared_norm)
                    .put<double>(g.max_abs)
                    .put<uint64_t>(g.nonfinite_count)
                    .put<int32_t>(g.first_nonfinite == INT_MAX ? -1 : g.first_nonfinite);
            send_frame(5, r);
        }
        validate_costs(cs, values, true);
        if (graph) graph->validate();
        for (int t = 0; t < layers; ++t)
            if (gs[t].nonfinite_count)
                throw Rejected(("non-finite weight gradient in layer " + std::to_string(t) + ", flattened index " +
                                std::to_string(gs[t].first_nonfinite) + "; no optimizer update performed for this iteration")
                                   .c_str());
        if (halves || fused_update) {  // the update went out behind the download
            require(updated == 1, "the update was not applied although the epoch passed its checks");
            if (method == 1) ++n.adam_step;
        } else if (method == 0) call(cpde_rprop(n.net));
        else {
            require(n.adam_step < uint64_t(INT_MAX), "Adam counter exceeds supported range");
            call(cpde_adam(n.net, int(++n.adam_step), n.learning_rate));
        }
        // The reference synchronises here (cuda/cpde_server.cu:409) only to
        // surface errors; every later host read (the next epoch's scalar
        // download, evaluation, snapshots, outputs) synchronises itself, so the
        // next epoch's launches queue behind the update instead.
        ++completed;
        ++n.updates;
        ++n.stage_done;
        n.remaining = epochs - completed;
        // the absolute update count survives short calls and checkpoints
        if (restore_every && n.updates % restore_every == 0) call(cpde_restore_steps(n.net, restore_step));
        const bool last = completed == epochs || (!ahead && stop.load());
        if (collect) report(0);
        if (eval && (completed % eval == 0 || last)) {
            evaluate_costs(n, ids, values, graph.get());
            report(1);
            last_eval = completed;
            if (outputs)
                for (uint64_t id : ids) {
                    CostRecord& c = cost(id);
                    const uint64_t out = evaluate(ni, c.input, c.width);
                    DataRecord& d = data(out);
                    std::vector<float> a(d.values.bytes / sizeof(float));
                    call(cpde_buffer_download(dev_, a.data(), d.values.ptr, d.values.bytes));
                    Frame r;
                    r.put<uint64_t>(id).put_array(a);
                    data_.erase(out);
                    send_frame(4, r);
                }
        }
        if (save && (completed % save == 0 || last)) {
            send_frame(3, snapshot(n));
            last_saved = completed;
        }
    }
    if (last_eval != completed) {
        evaluate_costs(n, ids, values, graph.get());
        report(1);
    }
    if (save && last_saved != completed) send_frame(3, snapshot(n));
    Frame result;
    const Frame meta = metadata(n);
    result.put<uint64_t>(completed).put<int32_t>(completed < epochs ? 1 : 0).put_array(meta.bytes);
    send_frame(0, result);
}

// op 90: the timing scope of the reference's benchmark build
// (docs/benchmarks/fourier-timing.patch:13-35): per step the cost slot is
// cleared and one forward + cost + weight-gradient pass runs; wall and device
// milliseconds per step for every batch, then the loss and the gradients.
void Server::timing(Frame& b, Frame& out) {
    const uint64_t ni = b.get<uint64_t>();
    NetRecord& n = net(ni);
    const uint64_t ci = b.get<uint64_t>();
    const int warm = b.get<int>(), iterations = b.get<int>(), batches = b.get<int>();
    b.end();
    require(warm >= 0 && iterations > 0 && batches > 0, "invalid benchmark controls");
    const std::vector<uint64_t> ids{ci};
    prepare_costs(n, ids, ni);
    CostRecord& c = cost(ci);
    auto step = [&]() {
        call(cpde_costs_begin(dev_, 1));
        bool first = true;
        pass(n, c, 0, first, Pass{true, true, nullptr, 0, INT_MAX, false});
    };
    for (int i = 0; i < warm; ++i) step();
    call(cpde_device_synchronize(dev_));
    std::vector<double> wall, gpu;
    for (int batch = 0; batch < batches; ++batch) {
        const auto t0 = std::chrono::steady_clock::now();
        call(cpde_mark(dev_, 0));
        for (int i = 0; i < iterations; ++i) step();
        call(cpde_mark(dev_, 1));
        float ms = 0;
        call(cpde_elapsed(dev_, 0, 1, &ms));
        const auto t1 = std::chrono::steady_clock::now();
        wall.push_back(std::chrono::duration<double, std::milli>(t1 - t0).count() / iterations);
        gpu.push_back(double(ms) / iterations);
    }
    out.put_array(wall).put_array(gpu);
    call(cpde_inspect_gradients(n.net));
    std::vector<cpde_cost_stats> cs;
    std::vector<cpde_gradient_stats> gs;
    download(1, n.transitions(), cs, gs);
    std::vector<double> values(1);
    validate_costs(cs, values, false);
    out.put<double>(values[0]);
    for (int t = 0; t < n.transitions(); ++t) {
        float* ptr = nullptr;
        int count = 0;
        call(cpde_net_state(n.net, t, cpde_net_active(n.net, t), &ptr, &count));
        std::vector<float> g(count);
        call(cpde_buffer_download(dev_, g.data(), ptr, g.size() * sizeof(float)));
        out.put_array(g);
    }
}

// op 7: matching (kind 0) or polynomial (kind 1) cost (cuda/cpde_server.cu:477-482).
uint64_t Server::create_cost(Frame& b) {
    auto c = std::make_unique<CostRecord>();
    c->net = b.get<uint64_t>();
    c->input = b.get<uint64_t>();
    c->target = b.get<uint64_t>();
    c->kind = b.get<int32_t>();
    const int chunk = b.get<int32_t>();
    c->rows = b.array<int>();
    NetRecord& n = net(c->net);
    DataRecord& d = data(c->input);
    require(d.channels == n.neurons.front(), "input channel mismatch");
    c->width = chunk ? std::min(chunk, d.samples) : d.samples;
    require(c->width > 0, "invalid chunk size");
    c->schema = make_schema(d, c->rows);
    const int outputs = n.neurons.back();
    if (c->kind == 0) {
        DataRecord& t = data(c->target);
        require(t.channels == outputs && t.samples == d.samples, "target shape mismatch");
        const auto target_rows = b.array<int>();
        c->weight_samples = b.get<int32_t>();
        const auto w = b.array<float>();
        require(target_rows.size() == c->rows.size() && (c->weight_samples == 1 || c->weight_samples == d.samples) &&
                    w.size() == c->rows.size() * size_t(c->weight_samples) * t.channels,
                "matching weight shape mismatch");
        for (int r : target_rows) require(r >= 0 && r < t.rows, "target derivative mismatch");
        for (float x : w) require(std::isfinite(x) && x >= 0, "invalid matching weight");
        c->target_rows.upload(dev_, target_rows);
        c->weights.upload(dev_, w);
    } else {
        require(c->kind == 1, "unknown cost kind");
        c->equations = b.get<int32_t>();
        const auto raw = b.array<int>();
        const auto co = b.array<float>(), rhs = b.array<float>(), w = b.array<float>();
        require(c->equations > 0 && raw.size() % 3 == 0 && co.size() == raw.size() / 3 * d.samples &&
                    rhs.size() == size_t(c->equations) * d.samples && w.size() == rhs.size(),
                "equation data shape mismatch");
        std::vector<cpde_poly_term> terms;
        const int comps = int(c->rows.size()) * outputs;
        for (size_t i = 0; i < raw.size(); i += 3) {
            require(raw[i] >= 0 && raw[i] < c->equations && raw[i + 1] >= 0 && raw[i + 1] < comps && raw[i + 2] >= -1 &&
                        raw[i + 2] < comps,
                    "invalid polynomial term");
            terms.push_back(cpde_poly_term{raw[i], raw[i + 1], raw[i + 2]});
        }
        for (float x : w) require(std::isfinite(x) && x >= 0, "invalid equation weight");
        for (float x : co) require(std::isfinite(x), "invalid coefficient");
        for (float x : rhs) require(std::isfinite(x), "invalid right-hand side");
        c->term_count = int(terms.size());
        c->terms.upload(dev_, terms);
        c->coefficients.upload(dev_, co);
        c->rhs.upload(dev_, rhs);
        c->weights.upload(dev_, w);
    }
    b.end();
    const uint64_t id = next_id_++;
    costs_[id] = std::move(c);
    return id;
}

// op 12: integral (expression) cost (cuda/cpde_server.cu:489-533): the
// derivative closure of the requested components, the IR remapped to the
// closure's rows, the kernel source generated and cached by its text.
uint64_t Server::create_integral(Frame& b) {
    auto c = std::make_unique<CostRecord>();
    c->kind = 2;
    c->net = b.get<uint64_t>();
    c->input = b.get<uint64_t>();
    const int chunk = b.get<int>();
    c->samples = b.get<int>();
    const auto raw = b.array<int>();
    const auto constants = b.array<double>();
    const int nfields = b.get<int>();
    const auto numeric = b.array<double>(), weights = b.array<double>();
    b.end();
    NetRecord& n = net(c->net);
    require(c->samples >= 0 && chunk >= 0 && nfields >= 0 && nfields <= 512 && weights.size() == size_t(c->samples) &&
                numeric.size() == size_t(nfields) * c->samples,
            "invalid integral field shape");
    require(!constants.empty() && constants.size() <= 512 && raw.size() == constants.size() * 3,
            "invalid expression IR size");
    const int outputs = n.neurons.back();
    if (c->samples) {
        DataRecord& d = data(c->input);
        require(d.channels == n.neurons.front() && d.samples == c->samples, "integral input shape mismatch");
        std::vector<int> requested;
        for (size_t i = 0; i < constants.size(); ++i)
            if (raw[3 * i] == kComponent) {
                const int component = raw[3 * i + 1];
                require(component >= 0 && int64_t(component) < int64_t(d.rows) * outputs,
                        "component outside derivative schema");
                requested.push_back(component / outputs);
            }
        // closure: the value row and every sub-derivative of a requested row
        for (int row : all_rows(d)) {
            bool needed = d.table.order(row) == 0;
            for (int target : requested) {
                bool below = true;
                for (int v = 0; v < d.table.variables && below; ++v) below = d.table.count(row, v) <= d.table.count(target, v);
                needed = needed || below;
            }
            if (needed) c->rows.push_back(row);
        }
        c->schema = make_schema(d, c->rows);
        c->width = chunk ? std::min(chunk, d.samples) : d.samples;
    } else {
        require(!c->input, "empty integral must not have input data");
        c->width = 0;
    }
    for (int i = 0; i < int(constants.size()); ++i) {
        const int op = raw[3 * i];
        int a = raw[3 * i + 1];
        const int mask = raw[3 * i + 2];
        require(op >= 0 && op <= kTanh && std::isfinite(constants[i]), "invalid expression node");
        if (op == kComponent) {
            require(a >= 0 && (mask == 0 || mask == 1), "invalid component");
            if (c->samples) {
                const auto row = std::find(c->rows.begin(), c->rows.end(), a / outputs);
                require(row != c->rows.end(), "component outside derivative closure");
                a = int(row - c->rows.begin()) * outputs + a % outputs;
            }
        }
        if (op == kField) require(a >= 0 && a < nfields, "invalid field index");
        if (op >= kAdd) {
            require(a >= 0 && a < i, "invalid expression dependency");
            if (op <= kDiv) require(mask >= 0 && mask < i, "invalid expression dependency");
        }
        c->ir.push_back(ExpressionNode{op, a, mask, constants[i]});
    }
    for (double x : numeric) require(std::isfinite(x), "nonfinite integral field");
    for (double x : weights) require(std::isfinite(x), "nonfinite quadrature weight");
    c->has_components = c->has_gradient = false;
    for (const auto& node : c->ir)
        if (node.op == kComponent) {
            c->has_components = true;
            if (node.b == 0) c->has_gradient = true;
        }
    c->source = expression_source(c->ir);
    c->fields.upload(dev_, numeric);
    c->quadrature.upload(dev_, weights);
    c->scratch.reset(dev_, size_t(std::max(1, c->width)) * (sizeof(double) + sizeof(int)));
    const uint64_t id = next_id_++;
    costs_[id] = std::move(c);
    return id;
}

void Server::command(uint32_t op, Frame& b, std::atomic<bool>& stop) {
    Frame out;
    if (op == 1) {
        b.end();
        // diagnostics | graphs | expressions | RPROP restore | wrapper initialisation
        out.put_string("CPDE/3").put<int32_t>(6).put<uint32_t>(31);
    } else if (op == 2) {
        const int d = b.get<int32_t>(), h = b.get<int32_t>(), w = b.get<int32_t>(), v = b.get<int32_t>();
        checked_size(d, h, w);
        require(v > 0 && v <= 26, "invalid variable count");
        const auto rows = b.array<int>();
        const auto a = b.array<float>();
        b.end();
        require(rows.size() == size_t(d) * (v + 1) && a.size() == size_t(d) * h * w, "data shape mismatch");
        open_device();  // every other command works on objects created here or by op 3
        auto rec = std::make_unique<DataRecord>();
        rec->rows = d;
        rec->channels = h;
        rec->samples = w;
        rec->table = Table{d, v, rows};
        rec->values.upload(dev_, a);
        const uint64_t id = next_id_++;
        data_[id] = std::move(rec);
        out.put<uint64_t>(id);
    } else if (op == 3) {
        const auto ns = b.array<int>(), ls = b.array<int>();
        require(ns.size() >= 2 && ns.size() <= 256 && ns.size() == ls.size(), "invalid architecture");
        for (size_t i = 0; i < ns.size(); ++i) require(ns[i] > 0 && (ls[i] == 0 || ls[i] == 1), "invalid layer");
        require(ls.front() == 1 && ls.back() == 1, "input and output layers must be linear");
        require(b.more(), "initial weights required; update the Python wrapper");
        std::vector<std::vector<float>> initial;
        for (size_t i = 1; i < ns.size(); ++i) {
            initial.push_back(b.array<float>());
            require(initial.back().size() == size_t(ns[i]) * (size_t(ns[i - 1]) + 1), "initial weight shape mismatch");
            for (float x : initial.back()) require(std::isfinite(x), "nonfinite initial weight");
        }
        b.end();
        open_device();
        std::vector<const float*> ptrs;
        for (const auto& w : initial) ptrs.push_back(w.data());
        auto rec = std::make_unique<NetRecord>();
        rec->neurons = ns;
        rec->linear = ls;
        call(cpde_net_create(dev_, int(ns.size()), ns.data(), ls.data(), ptrs.data(), &rec->net));
        const uint64_t id = next_id_++;
        nets_[id] = std::move(rec);
        out.put<uint64_t>(id);
    } else if (op == 4) {
        const uint64_t ni = b.get<uint64_t>(), di = b.get<uint64_t>();
        const int chunk = b.get<int32_t>();
        b.end();
        out.put<uint64_t>(evaluate(ni, di, chunk));
    } else if (op == 5) {
        DataRecord& d = data(b.get<uint64_t>());
        b.end();
        std::vector<float> a(d.values.bytes / sizeof(float));
        call(cpde_buffer_download(dev_, a.data(), d.values.ptr, d.values.bytes));
        out.put_array(a);
    } else if (op == 6) {
        DataRecord& d = data(b.get<uint64_t>());
        const auto a = b.array<float>();
        b.end();
        require(a.size() * sizeof(float) == d.values.bytes, "replacement data shape mismatch");
        call(cpde_buffer_upload(dev_, d.values.ptr, a.data(), d.values.bytes));
        ++d.version;
    } else if (op == 7) {
        out.put<uint64_t>(create_cost(b));
    } else if (op == 8) {
        train(b, stop, false);
        return;
    } else if (op == 9) {
        NetRecord& n = net(b.get<uint64_t>());
        b.end();
        out = snapshot(n);
    } else if (op == 10) {
        NetRecord& n = net(b.get<uint64_t>());
        restore(n, b);
    } else if (op == 11) {
        const int kind = b.get<int32_t>();
        const uint64_t id = b.get<uint64_t>();
        b.end();
        if (kind == 0) {
            for (auto& kv : costs_)
                require(kv.second->input != id && kv.second->target != id,
                        "data is retained by a cost; close that cost first");
            data_.erase(id);
        } else if (kind == 1) {
            for (auto& kv : costs_) require(kv.second->net != id, "network is retained by a cost; close that cost first");
            nets_.erase(id);
        } else if (kind == 2) {
            auto it = costs_.find(id);
            if (it != costs_.end()) {
                auto nt = nets_.find(it->second->net);
                if (nt != nets_.end()) nt->second->drop_retained(id);
            }
            costs_.erase(id);
        }
        else
            require(false, "invalid object kind");
    } else if (op == 12) {
        out.put<uint64_t>(create_integral(b));
    } else if (op == 13) {
        CostRecord& c = cost(b.get<uint64_t>());
        const bool compile = b.get<int>() != 0;
        b.end();
        require(c.kind == 2, "not a compiled expression cost");
        if (compile && !c.program) {
            auto it = programs_.find(c.source);
            if (it == programs_.end()) {
                cpde_program* prog = nullptr;
                std::vector<char> log(1 << 16);
                const int code = cpde_program_compile(dev_, c.source.c_str(), &prog, log.data(), log.size());
                c.log = log.data();
                call(code);
                it = programs_.emplace(c.source, prog).first;
            }
            c.program = it->second;
        }
        out.put_string(c.source).put_string(c.log);
    } else if (op == 14) {
        const uint64_t ni = b.get<uint64_t>();
        NetRecord& n = net(ni);
        const auto ids = b.array<uint64_t>();
        const bool gradient = b.get<int>() != 0;
        require(!ids.empty(), "cost graph needs at least one integral");
        GraphRecord graph;
        graph.read(dev_, b, int(ids.size()));
        b.end();
        prepare_costs(n, ids, ni);
        Frame saved;
        if (gradient) saved = snapshot(n);
        try {
            std::vector<double> values(ids.size());
            graph_pass(n, ids, graph, gradient);
            if (gradient) call(cpde_inspect_gradients(n.net));
            std::vector<cpde_cost_stats> cs;
            std::vector<cpde_gradient_stats> gs;
            download(int(ids.size()), gradient ? n.transitions() : 0, cs, gs, &graph);
            validate_costs(cs, values, false);
            graph.validate();
            out.put<double>(graph.host.value);
            if (gradient) {
                out.put<int>(n.transitions());
                for (int t = 0; t < n.transitions(); ++t) {
                    require(!gs[t].nonfinite_count, "nonfinite weight gradient during evaluation");
                    float* ptr = nullptr;
                    int count = 0;
                    call(cpde_net_state(n.net, t, cpde_net_active(n.net, t), &ptr, &count));
                    std::vector<float> g(count);
                    call(cpde_buffer_download(dev_, g.data(), ptr, g.size() * sizeof(float)));
                    out.put_array(g);
                }
            }
        } catch (...) {
            if (gradient) {
                saved.pos = 0;
                restore(n, saved);
            }
            throw;
        }
        if (gradient) {
            saved.pos = 0;
            restore(n, saved);
        }
    } else if (op == 15) {
        train(b, stop, true);
        return;
    } else if (op == 90) {
        timing(b, out);
    } else {
        require(false, "unknown command");
    }
    send_frame(0, out);
}

}  // namespace

int main(int argc, char** argv) {
    std::cout.rdbuf(std::cerr.rdbuf());
    int device = 0;
    if (argc == 3 && std::string(argv[1]) == "--device") device = std::stoi(argv[2]);
    std::mutex mutex;
    std::condition_variable ready;
    std::deque<Frame> queue;
    bool eof = false;
    std::atomic<bool> stop(false), training(false);
    std::string input_error;
    // reader: op 99 (stop) is handled here, everything else goes to the executor
    std::thread reader([&] {
        try {
            for (;;) {
                Frame f;
                if (!read_frame(f)) break;
                const uint32_t op = f.get<uint32_t>();
                if (op == 99) {
                    if (training.load()) stop.store(true);
                    continue;
                }
                if (op == 8 || op == 15) {
                    stop.store(false);
                    training.store(true);
                }
                const bool quit = op == 0;
                f.pos = 0;
                {
                    std::lock_guard<std::mutex> lock(mutex);
                    queue.push_back(std::move(f));
                }
                ready.notify_one();
                if (quit) break;
            }
        } catch (const std::exception& e) {
            input_error = e.what();
        }
        {
            std::lock_guard<std::mutex> lock(mutex);
            eof = true;
        }
        stop.store(true);
        ready.notify_one();
    });
    try {
        Server server(device);
        for (;;) {
            Frame f;
            {
                std::unique_lock<std::mutex> lock(mutex);
                ready.wait(lock, [&] { return eof || !queue.empty(); });
                if (queue.empty()) break;
                f = std::move(queue.front());
                queue.pop_front();
            }
            const uint32_t op = f.get<uint32_t>();
            if (op == 0) {
                send_frame(0);
                break;
            }
            try {
                server.command(op, f, stop);
            } catch (const std::exception& e) {
                Frame err;
                err.put_string(e.what());
                send_frame(1, err);
            }
            if (op == 8 || op == 15) training.store(false);
            stop.store(false);
        }
    } catch (const std::exception& e) {
        std::cerr << e.what() << std::endl;
    }
    reader.join();
    return input_error.empty() ? 0 : 1;
}
