// C ABI of the device library (include/cpde_hip.h).
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <string>

#include "common.hpp"

struct cpde_device_s : cpde::Device {};
struct cpde_net_s : cpde::Net {};
struct cpde_plan_s : cpde::Plan {};
struct cpde_stacks_s : cpde::Stacks {};
struct cpde_program_s : cpde::Program {};
struct cpde_replay_s {
    cpde::Device* dev = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t layout = 0;
    struct NetState {
        cpde::Net* net;
        std::vector<int> before, after;  // active gradient buffers when recorded, and after the recording
        uint64_t generation;
    };
    std::vector<NetState> nets;
};

namespace cpde {

// The no-allocation epoch's scratch (cpde_epoch_matching_static): one static
// device array that every GPU the library runs on holds until the process
// ends -- the launch's per-workgroup cost records (256-byte aligned), then its
// weight-gradient split partials.  Each kernel writes what it later reads
// within the same call, so nothing needs clearing between calls.  Host code
// never uses the array's name as an address: cpde_device_open takes this GPU's
// address with hipGetSymbolAddress (Device::static_scratch).
static __device__ __align__(256) unsigned char scratch[CPDE_STATIC_SCRATCH_BYTES];

static thread_local std::string last_error;

void set_error(const std::string& message) { last_error = message; }

void check_hip(hipError_t status, const char* what, const char* file, int line) {
    if (status == hipSuccess) return;
    char buf[512];
    std::snprintf(buf, sizeof buf, "%s:%d: %s failed: %s (%d)", file, line, what, hipGetErrorString(status),
                  int(status));
    throw device_error(buf);
}

static void flush_held(Device& d);

// Launch the held one-pass epoch and the waiting weight-gradient launch, if
// any; the reduction may wait on.
void flush_wgrad(Device& d) {
    flush_held(d);
    Device::PendingReduce& w = d.waiting;
    if (!w.open || !w.wgrad) return;
    w.wgrad = false;
    launch_wgrad_grouped(d, w.wa, w.flops);
}

// Launch the waiting gradient reduction, if any, after its weight gradient.
void flush_reduce(Device& d) {
    if (!d.waiting.open) return;
    flush_wgrad(d);
    d.waiting.open = false;
    d.waiting.partial_end = 0;
    launch_reduce_grouped(d, d.waiting.ra);
}

void sync_stream(Device& d, int site) {
    if (d.capturing)
        throw invalid("this call synchronises the device (it allocates, frees or reads back), which a capture "
                      "cannot record: run it once before cpde_capture_begin (api.hip:" + std::to_string(site) + ")");
    flush_reduce(d);
    HIP_CHECK(hipStreamSynchronize(d.stream));
}

TraceScope::TraceScope(Device& dev, int kind, double work) : d(dev) {
    if (!d.tracing) return;
    if (d.event_pool.size() < 2 * d.pending.size() + 2) {
        for (int i = 0; i < 64; ++i) {
            hipEvent_t e;
            HIP_CHECK(hipEventCreate(&e));
            d.event_pool.push_back(e);
        }
    }
    TraceRecord r{kind, work, d.event_pool[2 * d.pending.size()], d.event_pool[2 * d.pending.size() + 1]};
    HIP_CHECK(hipEventRecord(r.start, d.stream));
    index = int(d.pending.size());
    d.pending.push_back(r);
}

TraceScope::~TraceScope() {
    if (index >= 0) (void)hipEventRecord(d.pending[index].stop, d.stream);
}

void Device::fold_trace() {
    if (pending.empty()) return;
    sync_stream(*this, __LINE__);
    for (const auto& r : pending) {
        float ms = 0;
        HIP_CHECK(hipEventElapsedTime(&ms, r.start, r.stop));
        trace_ms[r.kind] += ms;
        trace_work[r.kind] += r.work;
        trace_launches[r.kind] += 1;
    }
    pending.clear();
}

void Device::reserve_costs(int costs) {
    require(costs >= 0, "invalid cost count");
    reserve_scalars(costs, grad_capacity);
}

void Device::reserve_grads(int layers) { reserve_scalars(cost_capacity, layers); }

// Grow the scalar block; slots already written keep their values.
void Device::reserve_scalars(int costs, int layers) {
    costs = std::max(costs, cost_capacity);
    layers = std::max(layers, grad_capacity);
    if (costs == cost_capacity && layers == grad_capacity && scalar_block) return;
    sync_stream(*this, __LINE__);
    const size_t cost_bytes = (sizeof(CostStats) * size_t(costs) + 255) / 256 * 256;
    const size_t grad_bytes = (sizeof(GradStats) * size_t(layers) + 255) / 256 * 256;
    const size_t bytes = cost_bytes + grad_bytes + sizeof(cpde_graph_summary);
    void *block = nullptr, *host = nullptr;
    HIP_CHECK(hipMalloc(&block, bytes));
    HIP_CHECK(hipHostMalloc(&host, bytes, hipHostMallocDefault));
    CostStats* c = static_cast<CostStats*>(block);
    GradStats* g = reinterpret_cast<GradStats*>(static_cast<char*>(block) + cost_bytes);
    auto* summary = reinterpret_cast<cpde_graph_summary*>(static_cast<char*>(block) + cost_bytes + grad_bytes);
    if (cost_capacity) HIP_CHECK(hipMemcpy(c, cost_totals, sizeof(CostStats) * cost_capacity, hipMemcpyDeviceToDevice));
    if (grad_capacity) HIP_CHECK(hipMemcpy(g, grad_totals, sizeof(GradStats) * grad_capacity, hipMemcpyDeviceToDevice));
    const cpde_graph_summary none{0.0, -1, 0};
    if (graph_summary)
        HIP_CHECK(hipMemcpy(summary, graph_summary, sizeof(cpde_graph_summary), hipMemcpyDeviceToDevice));
    else HIP_CHECK(hipMemcpy(summary, &none, sizeof(cpde_graph_summary), hipMemcpyHostToDevice));
    if (scalar_block) {
        ++layout;
        HIP_CHECK(hipFree(scalar_block));
    }
    if (host_block) HIP_CHECK(hipHostFree(host_block));
    scalar_block = block;
    host_block = host;
    cost_totals = c;
    grad_totals = g;
    host_costs = static_cast<CostStats*>(host);
    host_grads = reinterpret_cast<GradStats*>(static_cast<char*>(host) + cost_bytes);
    graph_summary = summary;
    host_graph_summary = reinterpret_cast<cpde_graph_summary*>(static_cast<char*>(host) + cost_bytes + grad_bytes);
    scalar_bytes = bytes;
    cost_capacity = costs;
    grad_capacity = layers;
}

// Grow the network's shared stack arena for a plan (Server::reserve,
// cuda/cpde_server.cu:128-147: contexts are views, growth invalidates them).
static void reserve_arena(Net& net, const Plan& p) {
    bool grow = false;
    for (int l = 0; l < net.layers; ++l)
        if (p.columns() * net.neurons[l] > net.capacity[l]) grow = true;
    if (!grow) return;
    require(!net.bound, "a stack set is bound to this network: unbind it before using another plan");
    sync_stream(*net.dev, __LINE__);
    ++net.dev->layout;
    for (int l = 0; l < net.layers; ++l) {
        const size_t need = std::max(net.capacity[l], p.columns() * net.neurons[l]);
        if (need == net.capacity[l]) continue;
        for (auto* v : {&net.z, &net.y, &net.g}) {
            if ((*v)[l]) HIP_CHECK(hipFree((*v)[l]));
            (*v)[l] = nullptr;
        }
        HIP_CHECK(hipMalloc(&net.z[l], need * sizeof(float)));
        if (!net.linear[l]) HIP_CHECK(hipMalloc(&net.y[l], need * sizeof(float)));
        if (l > 0) HIP_CHECK(hipMalloc(&net.g[l], need * sizeof(float)));
        net.capacity[l] = need;
    }
    ++net.generation;
}

// Swap the network's arena and the plan's input with the stack set's.
static void swap_binding(Net& n, Plan& p, Stacks& s) {
    std::swap(n.z, s.z);
    std::swap(n.y, s.y);
    std::swap(n.g, s.g);
    std::swap(n.capacity, s.capacity);
    std::swap(p.input, s.input);
    ++n.generation;
}

template <class F>
static int guarded(F body) {
    try {
        body();
        return CPDE_OK;
    } catch (const invalid& e) {
        set_error(e.what());
        return CPDE_EINVAL;
    } catch (const compile_error& e) {
        set_error(e.what());
        return CPDE_ECOMPILE;
    } catch (const device_error& e) {
        set_error(e.what());
        return CPDE_EDEVICE;
    } catch (const std::bad_alloc&) {
        set_error("host allocation failed");
        return CPDE_EDEVICE;
    } catch (const std::exception& e) {
        set_error(e.what());
        return CPDE_EDEVICE;
    }
}

// Re-raise the failure of a nested entry point with its own error class.
[[noreturn]] static void throw_code(int code) {
    const std::string message = last_error;
    if (code == CPDE_EINVAL) throw invalid(message);
    if (code == CPDE_ECOMPILE) throw compile_error(message);
    throw device_error(message);
}

// Layer l's values as the next transition reads them: the plan's activated
// input at layer 0, z of a linear layer, y otherwise.
static const float* activations(const Plan& p, int l) {
    const Net& net = *p.net;
    return l == 0 ? p.input : (net.linear[l] ? net.z[l] : net.y[l]);
}

// Device copy of a host row map; re-uploaded only when it changes (the map is
// fixed for a cost, so a training loop uploads it once).
static const int* plan_rows(Plan& p, const int* rows) {
    std::vector<int> map(rows, rows + p.rows);
    if (map != p.host_rows) {
        sync_stream(*p.net->dev, __LINE__);
        HIP_CHECK(hipMemcpy(p.dev_rows, map.data(), map.size() * sizeof(int), hipMemcpyHostToDevice));
        p.host_rows = map;
    }
    return p.dev_rows;
}

FusedModule::~FusedModule() {
    if (module) (void)hipModuleUnload(module);
}

ExpressionEpoch::~ExpressionEpoch() {
    if (module) (void)hipModuleUnload(module);
}

static int env_int(const char* name, int fallback) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : fallback;
}

// The layer-fused path covers sigmoid hidden layers between a linear input
// layer with few channels and a linear output layer with few outputs; other
// architectures use the table-driven kernels.  CPDE_FUSED=0 forces the latter.
static bool fused_eligible(const Net& n, const Plan& p) {
    if (!env_int("CPDE_FUSED", 1)) return false;
    const int L = n.layers;
    if (L < 3 || L - 1 > kMaxTransitions || p.rows > 64 || n.neurons[0] > 16) return false;
    for (int l = 1; l + 1 < L; ++l)
        if (n.linear[l] || n.neurons[l] > 256) return false;
    return n.neurons[L - 1] <= 8 && n.neurons[L - 1] <= n.neurons[L - 2];
}

static std::string device_arch(int ordinal) {
    hipDeviceProp_t prop;
    HIP_CHECK(hipGetDeviceProperties(&prop, ordinal));
    std::string arch = prop.gcnArchName;
    const size_t colon = arch.find(':');
    return colon == std::string::npos ? arch : arch.substr(0, colon);
}

// Host mirror of the network-fused kernels' argument block (fused.hip.in).
struct NetArgsHost {
    const float* W[32];
    float* Z[33];
    float* Y[33];
    float* G[33];
    const float* X;
    float* partial_in;
    float* partial_out;
    float* WT[32];
    float* partial_hidden[32];
    int block_offset, block_count;  // the pass's workgroups in the launch (count 0: the whole grid)
};

// Tuning of the fused kernels for a schema of `rows` derivative rows over chunks
// of `width` points (0: unknown) on `compute_units` CUs, for a network of
// `neurons`.  The network-fused kernels put as many points in a workgroup as
// fill one 32-column matrix-core tile (one point when the rows alone need a
// tile or more), but no more than spread the chunk over about one workgroup
// per CU.  Long grids of many-row points take two points per workgroup
// instead: each weight load feeds both, 2R rows pad to whole 16-column tiles
// (35 rows: 80 columns for two points against 48 for one), and the product
// tile is written over its operand tile, so a workgroup needs no more LDS
// than one point did.  That needs whole columns per composition lane (hidden
// widths above 64) and hidden widths that are multiples of 16.  Measured:
// 3->128^5->1 over 32,768 points 6.87 -> 5.79 ms per epoch, 2->256^4->1 over
// 65,536-point chunks 102.8 -> 95.4 ms; 2->128^4->1 at 729 points (under one
// workgroup per CU either way): two points per workgroup were slower.
static FusedTuning tuning(int rows, int width, int compute_units, const std::vector<int>& neurons) {
    FusedTuning t;
    int npb = rows <= 16 ? 32 / rows : 1;
    if (width > 0) {
        const int spread = std::max(1, env_int("CPDE_NET_MIN_BLOCKS", compute_units));
        npb = std::max(1, std::min(npb, (width + spread - 1) / spread));
        bool paired = rows > 16 && width >= 16 * compute_units && neurons.size() >= 3;
        for (size_t l = 1; l + 1 < neurons.size(); ++l) paired = paired && neurons[l] > 64 && neurons[l] % 16 == 0;
        if (paired) {
            npb = 2;
            t.alias = 1;
            t.col_tile = 16;
        }
    }
    // A value-only plan over at most one point per CU (a boundary leaf, which
    // the server's graph epochs pair with the interior's launch): eight points
    // per workgroup instead of one per CU -- eight columns still take one
    // 16-column tile, so a workgroup costs what one point's did, and the pair
    // launch carries an eighth of the waves.  Four waves, so that it still pairs.
    // Poisson graph epoch 0.0595 -> 0.0581 ms (one, two, four, eight and
    // sixteen points: 0.0595, 0.0593, 0.0587, 0.0581, 0.0587).
    const bool value_leaf = rows == 1 && width > 0 && width <= compute_units;
    if (value_leaf) npb = 8;
    t.points_per_block = std::max(1, env_int("CPDE_FUSED_POINTS", t.points_per_block));
    t.net_points_per_block = std::max(1, env_int("CPDE_NET_POINTS", npb));
    // A chunk of several-point workgroups that leaves CUs without a second
    // workgroup runs eight waves per workgroup: with one wave per SIMD the
    // matrix-core and load latencies of the layer chain have nothing to hide
    // behind.  2->128^4->1 over 729 points (three points per workgroup, 243
    // workgroups), ms per epoch at orders 0..3: 0.0416 -> 0.0409, 0.0454 ->
    // 0.0445, 0.0500 -> 0.0487, 0.0576 -> 0.0563.  With more workgroups than
    // CUs it was slower (order 4, 365 workgroups: 0.0700 -> 0.0742).
    if (width > 0 && rows <= 16 && npb > 1 && !value_leaf && (width + npb - 1) / npb <= compute_units)
        t.net_threads = 512;
    t.net_threads = env_int("CPDE_NET_THREADS", t.net_threads) == 512 ? 512 : 256;
    // The waves of a workgroup share a layer's products by output tile.  Where
    // 32x32 tiles of the narrowest hidden layer are fewer than the waves (a
    // 128-wide layer in eight waves, a 64-wide one in four), 16-column tiles
    // keep every wave busy.  2->128^4->1 over 729 points, ms per epoch with
    // 32 -> 16 columns: order 0 (eight waves) 0.0412 -> 0.0353, order 1
    // 0.0448 -> 0.0384, order 2 0.0491 -> 0.0467, order 3 0.0567 -> 0.0525;
    // order 4 (four waves, four tiles) 0.0700 -> 0.0719, so 32 stays there.
    // Columns that fit in 16 take 16 in any case: a 32-column tile would be
    // half padding.
    if (t.col_tile == 0 && t.net_points_per_block > 1 && neurons.size() >= 3) {
        int narrowest = neurons[1];
        for (size_t l = 1; l + 1 < neurons.size(); ++l) narrowest = std::min(narrowest, neurons[l]);
        const int columns = t.net_points_per_block * rows;
        const int col_tiles = (columns + 31) / 32;
        if (columns <= 16 || (narrowest + 31) / 32 * col_tiles < t.net_threads / 64) t.col_tile = 16;
    }
    // Whole compositions per lane, except for several-point workgroups of up
    // to 32 rows, where a split over lanes fills the waves: on the Taylor-scaled
    // rows of one point per workgroup the split only adds lanes that repeat the
    // jet (2->128^4->1 over 729 points, ms per epoch with a split of two against
    // none: order 5 (21 rows) 0.0936 / 0.0904, order 6 (28 rows) 0.1036 /
    // 0.0992; orders 1-4, several points per workgroup, within 0.3 %).
    const bool whole = rows > 32 || (rows > 16 && t.net_points_per_block == 1);
    t.max_split = std::max(1, env_int("CPDE_NET_SPLIT", whole ? 1 : t.max_split));
    t.max_split_adjoint = std::max(1, env_int("CPDE_NET_SPLIT_ADJOINT", t.max_split_adjoint));
    t.forward_blocks = std::max(1, env_int("CPDE_NET_FWD_OCC", t.forward_blocks));
    t.backward_blocks = std::max(1, env_int("CPDE_NET_BWD_OCC", t.backward_blocks));
    t.col_tile = env_int("CPDE_NET_COLTILE", t.col_tile);
    t.alias = env_int("CPDE_NET_ALIAS", t.alias);
    // Paired neuron blocks in the 16-column products (weight operands as
    // float2, one LDS operand read per two products), on wherever a layer's
    // width is a multiple of 32 per wave.  Measured, ms per epoch against the
    // single blocks: 2->128^4->1 order 6 at 729 points 0.0952 / 0.0963, order 5
    // 0.0879 / 0.0876, 3->128^5->1 order 4 at 32768 points 5.20 / 5.37.
    t.b_pairs = env_int("CPDE_NET_BPAIR", t.b_pairs);
    t.scaled = env_int("CPDE_SCALED", t.scaled) ? 1 : 0;
    // Diagnostics: clock stamps of the one-pass epoch's phases, written over
    // the output stack (cpde_amd/stamps.py reads them back).
    t.stamps = env_int("CPDE_PHASE_STAMPS", 0) ? 1 : 0;
    // One-pass epochs: wave priority by dispatch round (tier_priority in the
    // generated source; 0 turns it off).  It acts only where a launch has more
    // workgroups than CUs.
    t.tier_prio = env_int("CPDE_NET_TIER_PRIO", 125);
    t.tier_cus = compute_units;
    // Hidden weight-gradient partials from the network backward itself, on
    // request (CPDE_INKERNEL_WGRAD=1; hidden widths that are multiples of 16).
    // Measured on the Poisson graph epoch, whose 256-point one-row boundary
    // leaf runs 256 one-point workgroups: 0.0951 ms per epoch against 0.0932
    // with the separate weight-gradient launch (each workgroup writes a whole
    // 64 x 65 partial for its rank-one contribution), 0.107 with both leaves
    // in the kernel; so it is off by default.
    {
        bool widths16 = neurons.size() >= 4;
        for (size_t l = 1; l + 2 < neurons.size(); ++l)
            widths16 = widths16 && neurons[l] % 16 == 0 && neurons[l + 1] % 16 == 0;
        // 2: only where the partials stay small (blocks x hidden weights <= 2^20 floats)
        int hidden = 0;
        for (size_t l = 1; l + 2 < neurons.size(); ++l) hidden += neurons[l + 1] * (neurons[l] + 1);
        const long blocks = width > 0 ? (width + t.net_points_per_block - 1) / t.net_points_per_block : 1L << 30;
        const int mode = env_int("CPDE_INKERNEL_WGRAD", 0);
        t.inkernel_wgrad = widths16 && (mode == 1 || (mode == 2 && blocks * hidden <= (1L << 20))) ? 1 : 0;
    }
    return t;
}

static std::shared_ptr<FusedModule> load_fused(Device& d, const Tables& t, const std::vector<int>& neurons,
                                               int width) {
    const FusedTuning tune = tuning(t.rows, width, d.compute_units, neurons);
    const std::string src = fused_source(t, neurons, tune);
    for (auto& kv : d.fused_modules)
        if (kv.first == src) return kv.second;
    std::string log;
    const std::vector<char> code = compile_module(src, device_arch(d.ordinal), &log);
    auto m = std::make_shared<FusedModule>();
    m->points_per_block = tune.points_per_block;
    m->net_points_per_block = tune.net_points_per_block;
    m->net_threads = tune.net_threads;
    m->scaled = tune.scaled != 0;
    m->inkernel_wgrad = tune.inkernel_wgrad != 0;
    HIP_CHECK(hipModuleLoadData(&m->module, code.data()));
    HIP_CHECK(hipModuleGetFunction(&m->network_forward, m->module, "network_forward_k"));
    HIP_CHECK(hipModuleGetFunction(&m->network_backward, m->module, "network_backward_k"));
    HIP_CHECK(hipModuleGetFunction(&m->network_epoch, m->module, "network_epoch_k"));
    HIP_CHECK(hipModuleGetFunction(&m->input_layer, m->module, "input_layer_k"));
    HIP_CHECK(hipModuleGetFunction(&m->output_backward, m->module, "output_backward_k"));
    const int L = int(neurons.size());
    m->hidden_forward.assign(L, nullptr);
    m->hidden_backward.assign(L, nullptr);
    for (int k = 1; k + 2 < L; ++k) {
        HIP_CHECK(hipModuleGetFunction(&m->hidden_forward[k], m->module, ("hidden_forward_" + std::to_string(k)).c_str()));
        HIP_CHECK(
            hipModuleGetFunction(&m->hidden_backward[k], m->module, ("hidden_backward_" + std::to_string(k)).c_str()));
    }
    d.fused_modules.emplace_back(src, m);
    return m;
}

static void launch_module(Device& d, hipFunction_t f, unsigned gx, unsigned gy, void** args, unsigned threads = 256) {
    HIP_CHECK(hipModuleLaunchKernel(f, gx, gy, 1, threads, 1, 1, 0, d.stream, args, nullptr));
}

static NetArgsHost net_args(const Plan& p) {
    const Net& n = *p.net;
    NetArgsHost a{};
    for (int t = 0; t + 1 < n.layers; ++t) {
        a.W[t] = n.state[0][t];
        a.WT[t] = n.wt[t];
    }
    for (int l = 0; l < n.layers; ++l) {
        a.Z[l] = n.z[l];
        a.Y[l] = n.y[l];
        a.G[l] = n.g[l];
    }
    a.X = p.input;
    a.Z[0] = p.input;
    return a;
}

struct GradientPlan;
struct PartialSpace;
static GradientPlan network_gradients(Plan& p, int blocks, bool accumulate, const PartialSpace& space,
                                      NetArgsHost& a);

// Mode of the fused path: CPDE_FUSED=2 (default) network-fused, 1 layer-fused.
static bool network_mode() { return env_int("CPDE_FUSED", 2) >= 2; }

static void fused_forward(Plan& p) {
    Net& n = *p.net;
    Device& d = *n.dev;
    FusedModule& fm = *p.fused;
    const int L = n.layers, R = p.rows;
    int width = p.width;
    const double cols = double(p.columns());
    if (p.network) {
        NetArgsHost a = net_args(p);
        void* args[] = {&a, &width};
        double flops = 0;
        for (int t = 0; t + 1 < L; ++t) flops += 2.0 * n.neurons[t] * n.neurons[t + 1] * cols;
        TraceScope trace(d, kTraceNetworkForward, flops);
        launch_module(d, fm.network_forward, unsigned((width + fm.net_points_per_block - 1) / fm.net_points_per_block),
                      1, args, unsigned(fm.net_threads));
        n.wt_current = true;  // written by the forward's side job
        return;
    }
    {
        const float* W = n.state[0][0];
        const float* X = p.input;
        float* Z = n.z[1];
        float* Y = n.y[1];
        void* args[] = {&W, &X, &Z, &Y, &width};
        TraceScope trace(d, kTraceFusedInput, 4.0 * cols * (n.neurons[0] + 2 * n.neurons[1]));
        launch_module(d, fm.input_layer, unsigned((size_t(width) * n.neurons[1] + 255) / 256), 1, args);
    }
    for (int t = 1; t + 2 < L; ++t) {
        const float* W = n.state[0][t];
        const float* Yin = n.y[t];
        float* Z = n.z[t + 1];
        float* Y = n.y[t + 1];
        void* args[] = {&W, &Yin, &Z, &Y, &width};
        TraceScope trace(d, kTraceFusedForward, 2.0 * n.neurons[t] * n.neurons[t + 1] * cols);
        launch_module(d, fm.hidden_forward[t], unsigned((n.neurons[t + 1] + 63) / 64),
                      unsigned((width + fm.points_per_block - 1) / fm.points_per_block), args);
    }
    launch_output_forward(d, n.state[0][L - 2], n.y[L - 2], n.z[L - 1], n.neurons[L - 2], n.neurons[L - 1], R,
                          int(p.columns()));
}

// Weight gradients of every transition (dW_t = G_{t+1} Y_t^T plus the bias),
// split over the columns.  Transitions marked `external` have their split
// partials written by another kernel (the network-fused backward writes one
// per block for the input and output transitions); the others are computed by
// the grouped launch, whose matrix-core splits are shared out in proportion to
// each transition's 128x128 tiles, about one block per CU.
struct GradientPlan {
    WgradArgs wa{};
    ReduceArgs ra{};
    size_t offset[kMaxTransitions] = {};  // first partial of each transition (local index)
    double flops = 0;
    size_t total = 0;
    // partials in the network's own buffer: the network and the end of this
    // plan's floats there (its reduction may then wait, cpde_gradients_defer)
    Net* net = nullptr;
    size_t partial_end = 0;
};

// Where a gradient plan's split partials live: the network's own lazily grown
// buffer (base == nullptr), or a fixed region of `floats` floats that is never
// grown (the no-allocation epoch's static scratch).
struct PartialSpace {
    float* base = nullptr;
    size_t floats = 0;
};

// Weight-gradient tiles per compute unit the split-K decomposition aims for
// (CPDE_WGRAD_OCC; two, the kernel's occupancy, keep a second wave on every
// SIMD to cover the other's loads and barriers).
static int wgrad_blocks_per_cu() { return std::max(1, env_int("CPDE_WGRAD_OCC", 2)); }
// Direct tiles per CU the split-K aims for (CPDE_WGRAD_DIRECT_OCC).  One
// measured best on 2->128^4->1 over 729 points at every derivative order
// (fewer, longer splits: each tile's fixed cost of set-up, cross-wave sum and
// partial rows is paid half as often, and the reduction reads half the
// partials).  Epoch ms at orders 0..6, one tile per CU against two:
// 0.0416/0.0416, 0.0453/0.0475, 0.0499/0.0525, 0.0575/0.0597, 0.0701/0.0721,
// 0.0936/0.0954, 0.1033/0.1050; the Poisson graph epoch 0.0924 against 0.0943.
static int wgrad_direct_blocks_per_cu() { return std::max(1, env_int("CPDE_WGRAD_DIRECT_OCC", 1)); }

// The gradient plan of transitions [first, first + count), count at most
// kMaxTransitions (one grouped launch and one reduction); external_splits is
// indexed by the absolute transition.
// external_splits[t] > 0: transition t's partials come from the network
// kernels' workgroups (that many), split-minor, or split-major where
// external_major[t].
static GradientPlan plan_gradients(Plan& p, bool accumulate, const int* external_splits, int first, int count,
                                   PartialSpace space = {}, const unsigned char* external_major = nullptr) {
    Net& n = *p.net;
    Device& d = *n.dev;
    const int K = int(p.columns());
    const int T = count;
    GradientPlan g;
    // local transition k is the network's transition first + k
    auto thin = [&](int k) { return n.neurons[first + k + 1] <= 16 || n.neurons[first + k] <= 16; };
    // 128x128 tiles, or 64x64 when both widths are at most 64 -- or when the
    // 128x128 splits would be short (fewer than kWgradMinColumns columns each):
    // then four times the tiles give each split four times the columns, and
    // the split partials the reduction reads shrink fourfold
    bool small_tiles = false, direct = false;
    auto tile_of = [&](int k) {
        return direct || small_tiles || (n.neurons[first + k + 1] <= 64 && n.neurons[first + k] <= 64) ? 64 : 128;
    };
    auto tiles_of = [&](int k) {
        const int T0 = tile_of(k);
        return ((n.neurons[first + k + 1] + T0 - 1) / T0) * ((n.neurons[first + k] + T0 - 1) / T0);
    };
    auto count_tiles = [&] {
        int total = 0;
        for (int k = 0; k < T; ++k)
            if (!thin(k) && !external_splits[first + k]) total += tiles_of(k);
        return total;
    };
    // whole waves of tiles: a partial last wave would run alone for a whole split
    auto splits_for = [&](int tiles) {
        const int per_cu = direct ? wgrad_direct_blocks_per_cu() : wgrad_blocks_per_cu();
        return std::max(1, per_cu * d.compute_units / std::max(1, tiles));
    };
    int total_tiles = count_tiles();
    // 64x64 tiles fed straight from global memory, one per CU.  They beat the
    // LDS-staged tiles on long reductions too: 2->256^4->1 over 65,536-point
    // chunks 25.9 -> 24.8 ms of weight gradient per epoch, 3->128^5->1 over
    // 32,768 points 1.37 -> 1.27 ms.  CPDE_WGRAD_DIRECT=0 keeps the LDS-staged
    // tiles (128x128, or 64x64 where those splits would be short).
    const bool staged = env_int("CPDE_WGRAD_DIRECT", -1) == 0;
    if (total_tiles > 0 && !staged) {
        small_tiles = true;
        direct = true;
        total_tiles = count_tiles();
    } else if (total_tiles > 0 && K / splits_for(total_tiles) < kWgradMinColumns) {
        small_tiles = true;
        total_tiles = count_tiles();
    }
    g.wa.direct = direct ? 1 : 0;
    const int tile_splits = splits_for(total_tiles);
    g.wa.block_begin[0] = 0;
    g.ra.accumulate = accumulate ? 1 : 0;
    g.ra.transitions = T;
    g.ra.begin[0] = 0;
    g.ra.block_begin[0] = 0;
    int w = 0;
    for (int k = 0; k < T; ++k) {
        const int t = first + k;
        const int M = n.neurons[t + 1], N = n.neurons[t];
        int s = external_splits[t];
        if (!s) {
            const int tiles = thin(k) ? 1 : tiles_of(k);
            s = thin(k) ? 2 * d.compute_units : tile_splits;
            s = std::max(1, std::min(s, std::max(1, K / kWgradChunk)));
            int chunk = (K + s - 1) / s;
            chunk = (chunk + kWgradChunk - 1) / kWgradChunk * kWgradChunk;
            s = (K + chunk - 1) / chunk;
            g.wa.M[w] = M;
            g.wa.N[w] = N;
            g.wa.K[w] = K;
            g.wa.R[w] = p.rows;
            g.wa.kchunk[w] = chunk;
            g.wa.tile[w] = tile_of(k);
            g.wa.block_begin[w + 1] = g.wa.block_begin[w] + tiles * s;
            g.wa.G[w] = n.g[t + 1];
            g.wa.Y[w] = activations(p, t);
            g.flops += 2.0 * M * N * double(K);
            ++w;
        }
        g.offset[k] = g.total;
        g.total += size_t(s) * M * (N + 1);
        g.ra.M[k] = M;
        g.ra.N[k] = N;
        g.ra.splits[k] = s;
        g.ra.grad[k] = n.state[n.active[t]][t];
        g.ra.begin[k + 1] = g.ra.begin[k] + M * (N + 1);
        const bool minor = external_splits[t] && !(external_major && external_major[t]);
        g.ra.split_minor[k] = minor ? 1 : 0;
        g.ra.block_begin[k + 1] = g.ra.block_begin[k] + reduce_blocks(M * (N + 1), minor);
    }
    g.wa.transitions = w;
    float* base = space.base;
    if (base) {
        if (g.total > space.floats)
            throw invalid("the weight-gradient split partials need " + std::to_string(g.total * sizeof(float)) +
                          " bytes, beyond the " + std::to_string(space.floats * sizeof(float)) +
                          " bytes of static scratch left after the cost records");
    } else {
        // a waiting reduction of this network keeps the front of the buffer
        // when this plan's partials fit behind it and it can take a second
        // pass; otherwise it is launched, and the buffer grows so that the
        // next pass fits behind it
        size_t offset0 = 0, need = g.total;
        Device::PendingReduce& w = d.waiting;
        if (w.open) {
            const bool same = w.net == &n && !w.ra.second;
            if (same && w.partial_end + g.total <= n.partial_capacity) offset0 = w.partial_end;
            else {
                if (same) need = w.partial_end + g.total;
                flush_reduce(d);
            }
        }
        // while reductions are deferred, room for two consecutive passes side
        // by side, taken while no capture is open (a recorded epoch finds it)
        if (d.defer && !d.capturing) need = std::max(need, n.last_partials + g.total);
        n.last_partials = g.total;
        if (need > n.partial_capacity) {
            sync_stream(d, __LINE__);
            ++d.layout;
            if (n.partials) HIP_CHECK(hipFree(n.partials));
            n.partials = nullptr;
            HIP_CHECK(hipMalloc(&n.partials, need * sizeof(float)));
            n.partial_capacity = need;
        }
        base = n.partials + offset0;
        g.net = &n;
        g.partial_end = offset0 + g.total;
    }
    w = 0;
    for (int k = 0; k < T; ++k) {
        g.ra.partial[k] = base + g.offset[k];
        if (!external_splits[first + k]) g.wa.partial[w++] = base + g.offset[k];
    }
    return g;
}

// The gradient plan of a network backward over `blocks` workgroups: the input
// and output transitions' partials come from the workgroups (split-minor), and
// so do the hidden transitions' (split-major) when the module computes them in
// the kernel; the partial pointers go into `a`.
static GradientPlan network_gradients(Plan& p, int blocks, bool accumulate, const PartialSpace& space,
                                      NetArgsHost& a) {
    const int L = p.net->layers;
    int external[kMaxTransitions] = {};
    unsigned char major[kMaxTransitions] = {};
    external[0] = external[L - 2] = blocks;
    if (p.fused->inkernel_wgrad)
        for (int t = 1; t + 2 < L; ++t) {
            external[t] = blocks;
            major[t] = 1;
        }
    GradientPlan g = plan_gradients(p, accumulate, external, 0, L - 1, space, major);
    a.partial_in = const_cast<float*>(g.ra.partial[0]);
    a.partial_out = const_cast<float*>(g.ra.partial[L - 2]);
    for (int t = 1; t + 2 < L; ++t) a.partial_hidden[t] = const_cast<float*>(g.ra.partial[t]);
    return g;
}

// Whether reduction `g` can ride as the second pass of the waiting one: the
// same network, transitions, layouts and gradient buffers, accumulating onto
// the first pass's result, with room for its cost finishes.
static bool joins(const Device::PendingReduce& w, const GradientPlan& g) {
    const ReduceArgs &a = w.ra, &b = g.ra;
    if (!w.open || w.net != g.net || !g.net || a.second || a.with_graph || !b.accumulate ||
        a.transitions != b.transitions || a.costs + b.costs > kReduceCosts)
        return false;
    for (int k = 0; k < a.transitions; ++k)
        if (a.M[k] != b.M[k] || a.N[k] != b.N[k] || a.split_minor[k] != b.split_minor[k] || a.grad[k] != b.grad[k])
            return false;
    return true;
}

// `update`: the reduction also applies RPROP to the group's transitions
// (transitions [first, first + count) of `update`), whose gradients it
// completes; the caller flips the active buffers once every group is done.
// Otherwise, while the device defers reductions (cpde_gradients_defer), a
// pass's launches over partials in the network's own buffer wait: as the
// second pass of the waiting ones when it joins them (its weight-gradient
// tiles appended to the waiting launch's), else as the new waiting ones.
static void run_gradients(Device& d, const GradientPlan& g, Net* update = nullptr, int first = 0,
                          const Plan* plan = nullptr) {
    if (update || !d.defer || !g.net) {
        flush_reduce(d);
        if (g.wa.transitions > 0) launch_wgrad_grouped(d, g.wa, g.flops);
        if (update) launch_reduce_rprop(d, g.ra, *update, first);
        else launch_reduce_grouped(d, g.ra);
        return;
    }
    Device::PendingReduce& w = d.waiting;
    const bool tiles_fit = g.wa.transitions == 0 || !w.wgrad ||
                           (w.wa.direct == g.wa.direct && w.wa.transitions + g.wa.transitions <= kMaxTransitions);
    if (joins(w, g) && tiles_fit) {
        if (g.wa.transitions > 0) {
            if (!w.wgrad) {  // the waiting pass's tiles already ran
                w.wgrad = true;
                w.wa = g.wa;
                w.flops = g.flops;
            } else {
                WgradArgs& a = w.wa;
                const WgradArgs& b = g.wa;
                const int base = a.block_begin[a.transitions];
                for (int k = 0; k < b.transitions; ++k) {
                    const int i = a.transitions + k;
                    a.G[i] = b.G[k];
                    a.Y[i] = b.Y[k];
                    a.partial[i] = b.partial[k];
                    a.M[i] = b.M[k];
                    a.N[i] = b.N[k];
                    a.K[i] = b.K[k];
                    a.R[i] = b.R[k];
                    a.kchunk[i] = b.kchunk[k];
                    a.tile[i] = b.tile[k];
                    a.block_begin[i + 1] = base + b.block_begin[k + 1];
                }
                a.transitions += b.transitions;
                w.flops += g.flops;
            }
        }
        for (int k = 0; k < g.ra.transitions; ++k) {
            w.ra.partial2[k] = g.ra.partial[k];
            w.ra.splits2[k] = g.ra.splits[k];
        }
        w.ra.second = 1;
        for (int c = 0; c < g.ra.costs; ++c) {
            const int i = w.ra.costs++;
            w.ra.cost_partials[i] = g.ra.cost_partials[c];
            w.ra.cost_total[i] = g.ra.cost_total[c];
            w.ra.cost_count[i] = g.ra.cost_count[c];
            w.ra.cost_overwrite[i] = g.ra.cost_overwrite[c];
        }
        w.partial_end = g.partial_end;
        return;
    }
    flush_reduce(d);
    w.open = true;
    w.net = g.net;
    w.ra = g.ra;
    w.partial_end = g.partial_end;
    w.wgrad = g.wa.transitions > 0;
    w.wa = g.wa;
    w.flops = g.flops;
    w.plan = plan;
}

// Launch the waiting reduction when it reads `records` (which the caller is
// about to overwrite) or finishes a cost into `slot` (which the caller is
// about to finish into).
static void flush_if_reads(Device& d, const CostStats* records, int slot = -1) {
    const ReduceArgs& a = d.waiting.ra;
    if (!d.waiting.open) return;
    for (int c = 0; c < a.costs; ++c)
        if (a.cost_partials[c] == records || (slot >= 0 && a.cost_total[c] == d.cost_totals + slot))
            return flush_reduce(d);
}

// Host bookkeeping of an RPROP update launched as part of a reduction
// (launch_rprop does the same after its own launch).
static void rprop_done(Net& n) {
    for (auto& act : n.active) act = act == 1 ? 2 : 1;
    n.wt_current = true;
}

// Host mirror of the one-pass epoch's matching arguments (fused.hip.in MatchArgs).
struct MatchArgsHost {
    const float* target;
    const int* target_rows;
    const float* weights;
    CostStats* partials;
    int target_width, weight_samples, offset, valid, collect;
};

// Host mirror of the one-pass epoch's expression arguments (fused.hip.in ExpressionArgs).
struct ExpressionArgsHost {
    const double* fields;
    const double* weights;
    const double* multiplier;
    CostStats* partials;
    int samples, offset, valid, collect;
};

static int epoch_blocks(const Plan& p) {
    return (p.width + p.fused->net_points_per_block - 1) / p.fused->net_points_per_block;
}

// Whether the one-pass epoch applies: a network-fused plan whose chunk's
// workgroups are resident together (the saved kernel boundary matters); long
// grids keep separate launches, where the forward has its own, higher occupancy.
// CPDE_ONE_PASS=0 forces the separate launches (same kernels otherwise).
static bool one_pass_fits(const Plan& p) {
    return env_int("CPDE_ONE_PASS", 1) && p.fused && p.network && epoch_blocks(p) <= 4 * p.net->dev->compute_units;
}

// Rewrite the row-major weight copies of every hidden transition from the
// weights (one launch).
static void refresh_wt(Net& n) {
    std::vector<const float*> W;
    std::vector<float*> WT;
    std::vector<int> ni, no;
    for (int t = 1; t + 2 < n.layers; ++t) {
        W.push_back(n.state[0][t]);
        WT.push_back(n.wt[t]);
        ni.push_back(n.neurons[t]);
        no.push_back(n.neurons[t + 1]);
    }
    if (!W.empty()) launch_transpose(*n.dev, W.data(), WT.data(), ni.data(), no.data(), int(W.size()));
    n.wt_current = true;
}

// The per-workgroup cost records of a one-pass epoch.
// Two sets, used in turn: a pass's records stay intact while the next pass on
// the plan runs, so a waiting reduction can still finish the first pass's
// cost (cpde_gradients_defer).
static CostStats* epoch_records(Plan& p) {
    Device& d = *p.net->dev;
    const int blocks = epoch_blocks(p);
    if (blocks > p.epoch_capacity) {
        sync_stream(d, __LINE__);
        ++d.layout;
        if (p.epoch_partials) HIP_CHECK(hipFree(p.epoch_partials));
        p.epoch_partials = nullptr;
        HIP_CHECK(hipMalloc(&p.epoch_partials, 2 * sizeof(CostStats) * size_t(blocks)));
        p.epoch_capacity = blocks;
    }
    p.epoch_turn ^= 1;
    return p.epoch_partials + (p.epoch_turn ? p.epoch_capacity : 0);
}

// A plan's own layer stacks (Plan::own_*), shaped as its part of the arena:
// allocated on first use, outside captures, for plans of at most 256 MB of
// stacks.
static bool own_stacks(Plan& p) {
    if (!p.own_z.empty()) return true;
    const Net& n = *p.net;
    if (n.dev->capturing) return false;
    double bytes = 0;
    for (int l = 0; l < n.layers; ++l)
        bytes += 4.0 * p.columns() * n.neurons[l] * (1 + (n.linear[l] ? 0 : 1) + (l > 0 ? 1 : 0));
    if (bytes > 256.0 * 1048576.0) return false;
    std::vector<float*> z(n.layers, nullptr), y(n.layers, nullptr), g(n.layers, nullptr);
    try {
        for (int l = 0; l < n.layers; ++l) {
            const size_t need = p.columns() * n.neurons[l];
            HIP_CHECK(hipMalloc(&z[l], need * sizeof(float)));
            if (!n.linear[l]) HIP_CHECK(hipMalloc(&y[l], need * sizeof(float)));
            if (l > 0) HIP_CHECK(hipMalloc(&g[l], need * sizeof(float)));
        }
    } catch (...) {
        for (auto* v : {&z, &y, &g})
            for (float* q : *v) (void)hipFree(q);
        throw;
    }
    p.own_z = z;
    p.own_y = y;
    p.own_g = g;
    return true;
}

// The plan's own stacks in place of the network's arena for one pass.
struct OwnStacks {
    Net& n;
    Plan& p;
    bool on;
    OwnStacks(Net& net, Plan& plan, bool swapped) : n(net), p(plan), on(swapped) {}
    void swap() {
        std::swap(n.z, p.own_z);
        std::swap(n.y, p.own_y);
        std::swap(n.g, p.own_g);
        on = !on;
    }
    ~OwnStacks() {
        if (on) swap();
    }
};

// The held one-pass epoch (Device::held): an expression epoch issued while
// reductions are deferred, with everything its launch needs.
struct HeldEpoch {
    bool open = false;
    Plan* plan = nullptr;
    const Program* program = nullptr;
    hipFunction_t kernel = nullptr;  // its own epoch kernel, to launch it alone
    NetArgsHost a{};
    ExpressionArgsHost e{};
    int width = 0;
    unsigned blocks = 0, threads = 0;
    double flops = 0;
};

static bool epoch_pairs() { return env_int("CPDE_EPOCH_PAIRS", 1) != 0; }

// Launch the held epoch alone, if one is held.
static void flush_held(Device& d) {
    if (!d.held || !d.held->open) return;
    HeldEpoch& h = *d.held;
    h.open = false;
    void* args[] = {&h.a, &h.e, &h.width};
    TraceScope trace(d, kTraceNetworkEpoch, h.flops);
    launch_module(d, h.kernel, h.blocks, 1, args, h.threads);
}

// The kernel running the one-pass epochs of plans p0 (program g0) and p1
// (program g1) in one launch (compiled once, cached on disk and per device by
// source text, per plan pair by serial and program ids).  Null -- launch them
// apart -- while a capture is open and it is not loaded yet (loading a module
// is no launch to record), or when the pair does not compile or load (two
// programs may define the same name with C linkage): the failure is kept, so
// the pair is not tried again.
static hipFunction_t paired_epoch(const Plan& p0, const Program& g0, Plan& p1, const Program& g1) {
    for (const Plan::PairedEpoch& e : p1.paired_epochs)
        if (e.partner == p0.serial && e.partner_program == g0.id && e.program == g1.id)
            return e.epoch ? e.epoch->function : nullptr;
    Device& d = *p1.net->dev;
    if (d.capturing) return nullptr;
    const FusedTuning u0 = tuning(p0.tables.rows, p0.width, d.compute_units, p0.net->neurons);
    const FusedTuning u1 = tuning(p1.tables.rows, p1.width, d.compute_units, p1.net->neurons);
    std::shared_ptr<ExpressionEpoch> e;
    try {
        const std::string src =
            expression_pair_source(p0.tables, u0, g0.source, p1.tables, u1, g1.source, p1.net->neurons);
        for (auto& kv : d.expression_epochs)
            if (kv.first == src) e = kv.second;
        if (!e) {
            std::string log;
            const std::vector<char> code = compile_module(src, device_arch(d.ordinal), &log);
            auto loaded = std::make_shared<ExpressionEpoch>();
            HIP_CHECK(hipModuleLoadData(&loaded->module, code.data()));
            HIP_CHECK(hipModuleGetFunction(&loaded->function, loaded->module, "network_epoch_pair_k"));
            d.expression_epochs.emplace_back(src, loaded);
            e = loaded;
        }
    } catch (const std::exception&) {
        e = nullptr;
    }
    p1.paired_epochs.push_back(Plan::PairedEpoch{p0.serial, g0.id, g1.id, e});
    return e ? e->function : nullptr;
}

// Launch a one-pass expression epoch of plan p (program g; kernel arguments a,
// e, width over `blocks` workgroups) as the reductions are deferred: held back
// when nothing is held, or in one launch with the held epoch when that is of
// another plan over the same network and this pass runs on stacks of its own
// (so the two write different stacks, and different partials, as the held
// pass's weight gradient is waiting).  False: launch it alone (the held epoch,
// if any, has gone out).  Only epochs whose cost finish rides in the gradient
// reduction are held, so nothing launched in between reads their records.
static bool pair_or_hold(Plan& p, const Program* g, hipFunction_t kernel, NetArgsHost& a, ExpressionArgsHost* e,
                         int width, int blocks, double flops, bool own) {
    Device& d = *p.net->dev;
    const unsigned threads = unsigned(p.fused->net_threads);
    if (d.held && d.held->open) {
        HeldEpoch& h = *d.held;
        const hipFunction_t pair = g && epoch_pairs() && own && h.plan != &p && h.plan->net == p.net &&
                                           h.threads == threads
                                       ? paired_epoch(*h.plan, *h.program, p, *g)
                                       : nullptr;
        if (pair) {
            h.open = false;
            h.a.block_offset = 0;
            h.a.block_count = int(h.blocks);
            a.block_offset = int(h.blocks);
            a.block_count = blocks;
            void* args[] = {&h.a, &h.e, &h.width, &a, e, &width};
            TraceScope trace(d, kTraceNetworkEpoch, h.flops + flops);
            launch_module(d, pair, h.blocks + unsigned(blocks), 1, args, threads);
            return true;
        }
        flush_held(d);
    }
    if (!g || !epoch_pairs() || !d.defer || blocks > kMaxCostBlocks) return false;
    if (!d.held) d.held = std::make_shared<HeldEpoch>();
    HeldEpoch& h = *d.held;
    h.open = true;
    h.plan = &p;
    h.program = g;
    h.kernel = kernel;
    h.a = a;
    h.e = *e;
    h.width = width;
    h.blocks = unsigned(blocks);
    h.threads = threads;
    h.flops = flops;
    return true;
}

// Forward, cost and backward of one chunk in one network-fused launch of
// `kernel` (arguments: the network, `cost_args`, the chunk width), then the
// cost's fixed-order finish and the weight-gradient contraction.  `records`
// holds the launch's per-workgroup cost records; `space` says where the
// weight-gradient split partials go.  Everything that can be refused is
// checked before the first launch.
static void one_pass_epoch(Plan& p, hipFunction_t kernel, void* cost_args, CostStats* records, int cost_index,
                           bool accumulate, PartialSpace space = {}, bool update = false,
                           const Program* program = nullptr) {
    Net& n = *p.net;
    Device& d = *n.dev;
    const int L = n.layers;
    int width = p.width;
    const double cols = double(p.columns());
    const int blocks = epoch_blocks(p);
    // a held epoch this one cannot join goes out before anything of this one
    if (d.held && d.held->open && (!program || !epoch_pairs() || d.held->plan == &p || d.held->plan->net != &n))
        flush_held(d);
    flush_if_reads(d, records, cost_index);  // the kernel rewrites this plan's records
    // Behind a waiting weight gradient that reads another plan's stacks in the
    // arena, this pass runs on stacks of its own, so that both passes' tiles
    // go out in one launch; a waiting gradient this pass would overwrite goes
    // out now.
    OwnStacks own(n, p, false);
    {
        const Device::PendingReduce& w = d.waiting;
        if (w.open && w.wgrad && w.net == &n) {
            if (!w.ra.second && !space.base && !update && w.plan != &p && !n.bound && own_stacks(p)) own.swap();
            else flush_wgrad(d);
        }
    }
    NetArgsHost a = net_args(p);
    GradientPlan g = network_gradients(p, blocks, accumulate, space, a);
    // the backward half reads the row-major weight copies of every hidden
    // transition, which no workgroup of the same launch may still be writing;
    // RPROP and Adam keep them current between epochs
    if (!n.wt_current) refresh_wt(n);
    void* args[] = {&a, cost_args, &width};
    double flops = 0;
    for (int t = 0; t + 1 < L; ++t) flops += 2.0 * n.neurons[t] * n.neurons[t + 1] * cols;
    for (int t = 1; t + 1 < L; ++t) flops += 2.0 * n.neurons[t] * n.neurons[t + 1] * cols;
    // an expression epoch (`program`) may wait for, or join, another plan's
    if (!pair_or_hold(p, program, kernel, a, static_cast<ExpressionArgsHost*>(cost_args), width, blocks, flops,
                      own.on)) {
        TraceScope trace(d, kTraceNetworkEpoch, flops);
        launch_module(d, kernel, unsigned(blocks), 1, args, unsigned(p.fused->net_threads));
    }
    if (blocks <= kMaxCostBlocks) {  // the cost's finish rides in the gradient reduction launch
        g.ra.costs = 1;
        g.ra.cost_partials[0] = records;
        g.ra.cost_total[0] = d.cost_totals + cost_index;
        g.ra.cost_count[0] = blocks;
        g.ra.cost_overwrite[0] = d.take_fresh(cost_index) ? 1 : 0;
    } else {
        launch_finish_cost(d, records, blocks, cost_index);
    }
    run_gradients(d, g, update ? &n : nullptr, 0, &p);
    if (update) rprop_done(n);
}

// The plan's one-pass epoch kernel for an expression program: the program's
// source compiled together with the plan's network kernels (cached on disk and
// per device by source text, per plan by program id).
static hipFunction_t expression_epoch(Plan& p, const Program& program) {
    for (auto& kv : p.expression_epochs)
        if (kv.first == program.id) return kv.second->function;
    Device& d = *p.net->dev;
    const FusedTuning tune = tuning(p.tables.rows, p.width, d.compute_units, p.net->neurons);
    const std::string src = expression_epoch_source(p.tables, p.net->neurons, tune, program.source);
    std::shared_ptr<ExpressionEpoch> e;
    for (auto& kv : d.expression_epochs)
        if (kv.first == src) e = kv.second;
    if (!e) {
        std::string log;
        const std::vector<char> code = compile_module(src, device_arch(d.ordinal), &log);
        e = std::make_shared<ExpressionEpoch>();
        HIP_CHECK(hipModuleLoadData(&e->module, code.data()));
        HIP_CHECK(hipModuleGetFunction(&e->function, e->module, "network_epoch_expression_k"));
        d.expression_epochs.emplace_back(src, e);
    }
    p.expression_epochs.emplace_back(program.id, e);
    return e->function;
}

// Every transition's weight gradient, kMaxTransitions transitions per grouped
// launch and reduction (the groups reuse the partials in stream order).
static void weight_gradients(Plan& p, bool accumulate) {
    const int T = p.net->layers - 1;
    const std::vector<int> none(T, 0);
    for (int first = 0; first < T; first += kMaxTransitions)
        run_gradients(*p.net->dev,
                      plan_gradients(p, accumulate, none.data(), first, std::min(kMaxTransitions, T - first)),
                      nullptr, 0, &p);
}

static void fused_backward(Plan& p, bool accumulate) {
    Net& n = *p.net;
    Device& d = *n.dev;
    FusedModule& fm = *p.fused;
    const int L = n.layers;
    int width = p.width;
    const double cols = double(p.columns());
    if (p.network) {
        const int blocks = (width + fm.net_points_per_block - 1) / fm.net_points_per_block;
        NetArgsHost a = net_args(p);
        const GradientPlan g = network_gradients(p, blocks, accumulate, PartialSpace{}, a);
        void* args[] = {&a, &width};
        double flops = 0;
        for (int t = 1; t + 1 < L; ++t) flops += 2.0 * n.neurons[t] * n.neurons[t + 1] * cols;
        {
            TraceScope trace(d, kTraceNetworkBackward, flops);
            launch_module(d, fm.network_backward, unsigned(blocks), 1, args, unsigned(fm.net_threads));
        }
        run_gradients(d, g, nullptr, 0, &p);
        return;
    }
    {
        const int NIo = n.neurons[L - 2], NOo = n.neurons[L - 1];
        const float* W = n.state[0][L - 2];
        const float* G = n.g[L - 1];
        const float* Zl = n.z[L - 2];
        float* Gl = n.g[L - 2];
        void* args[] = {&W, &G, &Zl, &Gl, &width};
        TraceScope trace(d, kTraceFusedOutput, 4.0 * cols * (3.0 * NIo + NOo));
        launch_module(d, fm.output_backward, unsigned((size_t(width) * NIo + 255) / 256), 1, args);
    }
    for (int t = L - 3; t >= 1; --t) {
        const float* W = n.state[0][t];
        const float* Gnext = n.g[t + 1];
        const float* Zl = n.z[t];
        float* Gl = n.g[t];
        void* args[] = {&W, &Gnext, &Zl, &Gl, &width};
        TraceScope trace(d, kTraceFusedBackward, 2.0 * n.neurons[t] * n.neurons[t + 1] * cols);
        launch_module(d, fm.hidden_backward[t], unsigned((n.neurons[t] + 63) / 64),
                      unsigned((width + fm.points_per_block - 1) / fm.points_per_block), args);
    }
    weight_gradients(p, accumulate);
}

}  // namespace cpde

using namespace cpde;

extern "C" {

const char* cpde_last_error(void) { return cpde::last_error.c_str(); }

int cpde_device_open(int ordinal, cpde_device** out) {
    return guarded([&] {
        require(out != nullptr, "null output");
        int count = 0;
        HIP_CHECK(hipGetDeviceCount(&count));
        require(ordinal >= 0 && ordinal < count, "invalid device ordinal");
        HIP_CHECK(hipSetDevice(ordinal));
        auto d = std::make_unique<cpde_device>();
        d->ordinal = ordinal;
        hipDeviceProp_t prop;
        HIP_CHECK(hipGetDeviceProperties(&prop, ordinal));
        d->compute_units = prop.multiProcessorCount;
        HIP_CHECK(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking));
        {
            // this GPU's address of the static scratch (the device is current)
            void* ptr = nullptr;
            const hipError_t status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
            if (status == hipSuccess && ptr) d->static_scratch = static_cast<unsigned char*>(ptr);
            else d->static_scratch_error = std::string("hipGetSymbolAddress failed: ") + hipGetErrorString(status);
        }
        HIP_CHECK(hipMalloc(&d->cost_blocks, sizeof(CostStats) * kMaxCostBlocks));
        HIP_CHECK(hipMalloc(&d->update_verdict, sizeof(int)));
        HIP_CHECK(hipMemset(d->update_verdict, 0, sizeof(int)));
        for (auto& e : d->marks) HIP_CHECK(hipEventCreate(&e));
        HIP_CHECK(hipEventCreateWithFlags(&d->copied, hipEventDisableTiming));
        d->reserve_scalars(8, 8);
        HIP_CHECK(hipHostMalloc(&d->host_summary, sizeof(cpde_graph_summary), hipHostMallocDefault));
        *out = d.release();
    });
}

int cpde_device_close(cpde_device* dev) {
    return guarded([&] {
        if (!dev) return;
        if (dev->capturing) {  // an open capture is abandoned
            hipGraph_t graph = nullptr;
            (void)hipStreamEndCapture(dev->stream, &graph);
            if (graph) (void)hipGraphDestroy(graph);
            dev->capturing = false;
        }
        (void)hipStreamSynchronize(dev->stream);
        for (auto& e : dev->marks) (void)hipEventDestroy(e);
        if (dev->copied) (void)hipEventDestroy(dev->copied);
        for (auto& e : dev->event_pool) (void)hipEventDestroy(e);
        (void)hipFree(dev->cost_blocks);
        (void)hipFree(dev->update_verdict);
        (void)hipFree(dev->scalar_block);
        (void)hipHostFree(dev->host_block);
        (void)hipHostFree(dev->host_summary);
        (void)hipStreamDestroy(dev->stream);
        delete dev;
    });
}

int cpde_device_synchronize(cpde_device* dev) {
    return guarded([&] { sync_stream(*dev, __LINE__); });
}

int cpde_device_info(cpde_device* dev, char* name, size_t capacity, int* compute_units) {
    return guarded([&] {
        hipDeviceProp_t prop;
        HIP_CHECK(hipGetDeviceProperties(&prop, dev->ordinal));
        if (name && capacity) {
            std::snprintf(name, capacity, "%s (%s)", prop.name, prop.gcnArchName);
        }
        if (compute_units) *compute_units = prop.multiProcessorCount;
    });
}

int cpde_buffer_alloc(cpde_device* dev, size_t bytes, void** out) {
    return guarded([&] {
        require(out != nullptr, "null output");
        *out = nullptr;
        if (bytes) HIP_CHECK(hipMalloc(out, bytes));
        (void)dev;
    });
}

int cpde_buffer_free(cpde_device* dev, void* ptr) {
    return guarded([&] {
        if (!ptr) return;
        sync_stream(*dev, __LINE__);
        ++dev->layout;
        HIP_CHECK(hipFree(ptr));
    });
}

int cpde_buffer_upload(cpde_device* dev, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        flush_reduce(*dev);
        if (!bytes) return;
        HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, dev->stream));
        sync_stream(*dev, __LINE__);
    });
}

int cpde_buffer_download(cpde_device* dev, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        flush_reduce(*dev);
        if (!bytes) return;
        HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, dev->stream));
        sync_stream(*dev, __LINE__);
    });
}

int cpde_buffer_copy(cpde_device* dev, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        flush_reduce(*dev);
        if (!bytes) return;
        HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, dev->stream));
    });
}

// ---- network --------------------------------------------------------------------------
int cpde_net_create(cpde_device* dev, int layers, const int* neurons, const int* linear, const float* const* initial,
                    cpde_net** out) {
    return guarded([&] {
        require(out && neurons && linear, "null argument");
        require(layers >= 2 && layers <= 256, "invalid architecture");
        for (int l = 0; l < layers; ++l) require(neurons[l] > 0 && (linear[l] == 0 || linear[l] == 1), "invalid layer");
        require(linear[0] == 1 && linear[layers - 1] == 1, "input and output layers must be linear");
        auto n = std::make_unique<cpde_net>();
        n->dev = dev;
        n->layers = layers;
        n->neurons.assign(neurons, neurons + layers);
        n->linear.assign(linear, linear + layers);
        const int T = layers - 1;
        for (auto& s : n->state) s.assign(T, nullptr);
        n->wt.assign(T, nullptr);
        n->active.assign(T, 1);
        n->z.assign(layers, nullptr);
        n->y.assign(layers, nullptr);
        n->g.assign(layers, nullptr);
        n->capacity.assign(layers, 0);
        for (int t = 0; t < T; ++t) {
            const size_t count = n->param_count(t);
            for (int b = 0; b < 4; ++b) HIP_CHECK(hipMalloc(&n->state[b][t], count * sizeof(float)));
            HIP_CHECK(hipMalloc(&n->wt[t], size_t(n->neurons[t]) * n->neurons[t + 1] * sizeof(float)));
            if (initial && initial[t])
                HIP_CHECK(hipMemcpyAsync(n->state[0][t], initial[t], count * sizeof(float), hipMemcpyHostToDevice,
                                         dev->stream));
            else
                HIP_CHECK(hipMemsetAsync(n->state[0][t], 0, count * sizeof(float), dev->stream));
            HIP_CHECK(hipMemsetAsync(n->state[1][t], 0, count * sizeof(float), dev->stream));
            HIP_CHECK(hipMemsetAsync(n->state[2][t], 0, count * sizeof(float), dev->stream));
            launch_fill(*dev, n->state[3][t], count, 0.002f);
        }
        dev->reserve_grads(T);
        sync_stream(*dev, __LINE__);
        dev->nets.push_back(n.get());
        *out = n.release();
    });
}

int cpde_net_destroy(cpde_net* net) {
    return guarded([&] {
        if (!net) return;
        sync_stream(*net->dev, __LINE__);
        if (net->bound) {  // the arena's buffers go back to the network before it frees them
            swap_binding(*net, *net->bound->plan, *net->bound);
            net->bound = nullptr;
        }
        auto& live = net->dev->nets;
        live.erase(std::remove(live.begin(), live.end(), static_cast<Net*>(net)), live.end());
        ++net->dev->layout;
        for (auto& s : net->state)
            for (float* p : s) (void)hipFree(p);
        for (float* p : net->wt) (void)hipFree(p);
        for (auto* v : {&net->z, &net->y, &net->g})
            for (float* p : *v) (void)hipFree(p);
        (void)hipFree(net->partials);
        delete net;
    });
}

int cpde_net_state(cpde_net* net, int transition, int buffer, float** device_ptr, int* count) {
    return guarded([&] {
        flush_reduce(*net->dev);
        require(transition >= 0 && transition < net->layers - 1 && buffer >= 0 && buffer < 4, "invalid state buffer");
        if (buffer == 0) net->wt_current = false;  // the caller may write the weights
        if (device_ptr) *device_ptr = net->state[buffer][transition];
        if (count) *count = net->param_count(transition);
    });
}

int cpde_net_active(cpde_net* net, int transition) {
    if (!net || transition < 0 || transition >= net->layers - 1) return -1;
    return net->active[transition];
}

int cpde_net_set_active(cpde_net* net, int transition, int active) {
    return guarded([&] {
        flush_reduce(*net->dev);
        require(transition >= 0 && transition < net->layers - 1 && (active == 1 || active == 2),
                "invalid active gradient buffer");
        net->active[transition] = active;
    });
}

uint64_t cpde_net_generation(cpde_net* net) { return net ? net->generation : 0; }

// ---- plans ----------------------------------------------------------------------------
int cpde_plan_create(cpde_net* net, int rows, int variables, const int* table, int width, int backward,
                     cpde_plan** out) {
    return guarded([&] {
        require(net && table && out, "null argument");
        require(width > 0, "invalid chunk size");
        static std::atomic<uint64_t> serials{0};
        auto p = std::make_unique<cpde_plan>();
        p->serial = ++serials;
        p->net = net;
        p->rows = rows;
        p->variables = variables;
        p->width = width;
        p->backward = backward ? 1 : 0;
        p->tables = build_tables(rows, variables, table);
        for (int l = 0; l < net->layers; ++l)
            require(double(width) * rows * net->neurons[l] < double(1ull << 40), "context exceeds device capacity");
        // kernels index a chunk's (point, row) and (point, neuron) pairs, and
        // the weight gradient its R x width columns, in 32 bits
        require(double(width) * rows < double(1 << 30), "chunk too large: rows x width must stay below 2^30");
        for (int l = 0; l < net->layers; ++l)
            require(double(width) * net->neurons[l] < double(1 << 30),
                    "chunk too large: width x neurons must stay below 2^30");
        std::vector<int> blob = p->tables.words;
        blob.insert(blob.end(), p->tables.fwd_offset.begin(), p->tables.fwd_offset.end());
        HIP_CHECK(hipMalloc(&p->dev_tables, blob.size() * sizeof(int)));
        HIP_CHECK(hipMalloc(&p->dev_rows, size_t(rows) * sizeof(int)));
        HIP_CHECK(hipMalloc(&p->input, p->columns() * net->neurons[0] * sizeof(float)));
        launch_fill(*net->dev, p->input, p->columns() * net->neurons[0], 0.0f);
        HIP_CHECK(hipMemcpyAsync(p->dev_tables, blob.data(), blob.size() * sizeof(int), hipMemcpyHostToDevice,
                                 net->dev->stream));
        reserve_arena(*net, *p);
        if (fused_eligible(*net, *p)) {
            p->fused = load_fused(*net->dev, p->tables, net->neurons, width);
            p->network = network_mode();
        }
        sync_stream(*net->dev, __LINE__);
        *out = p.release();
    });
}

int cpde_plan_destroy(cpde_plan* plan) {
    return guarded([&] {
        if (!plan) return;
        Net& n = *plan->net;
        sync_stream(*n.dev, __LINE__);
        if (n.bound && n.bound->plan == plan) {
            swap_binding(n, *plan, *n.bound);
            n.bound = nullptr;
        }
        ++n.dev->layout;
        (void)hipFree(plan->dev_tables);
        (void)hipFree(plan->dev_rows);
        (void)hipFree(plan->epoch_partials);
        (void)hipFree(plan->input);
        for (auto* v : {&plan->own_z, &plan->own_y, &plan->own_g})
            for (float* q : *v) (void)hipFree(q);
        delete plan;
    });
}

int cpde_stacks_create(cpde_plan* plan, cpde_stacks** out) {
    return guarded([&] {
        require(plan && out, "null argument");
        Net& n = *plan->net;
        auto s = std::make_unique<cpde_stacks>();
        s->plan = plan;
        s->z.assign(n.layers, nullptr);
        s->y.assign(n.layers, nullptr);
        s->g.assign(n.layers, nullptr);
        s->capacity.assign(n.layers, 0);
        try {
            for (int l = 0; l < n.layers; ++l) {
                const size_t need = plan->columns() * n.neurons[l];
                HIP_CHECK(hipMalloc(&s->z[l], need * sizeof(float)));
                if (!n.linear[l]) HIP_CHECK(hipMalloc(&s->y[l], need * sizeof(float)));
                if (l > 0) HIP_CHECK(hipMalloc(&s->g[l], need * sizeof(float)));
                s->capacity[l] = need;
            }
            HIP_CHECK(hipMalloc(&s->input, plan->columns() * n.neurons[0] * sizeof(float)));
        } catch (...) {
            for (auto* v : {&s->z, &s->y, &s->g})
                for (float* q : *v) (void)hipFree(q);
            (void)hipFree(s->input);
            throw;
        }
        *out = s.release();
    });
}

int cpde_plan_bind(cpde_plan* plan, cpde_stacks* stacks) {
    return guarded([&] {
        require(plan, "null argument");
        flush_wgrad(*plan->net->dev);  // this call writes stacks a waiting launch may read
        Net& n = *plan->net;
        if (n.bound) {  // unbind whatever is bound: the set goes back to its own pointers
            Stacks& b = *n.bound;
            swap_binding(n, *b.plan, b);
            n.bound = nullptr;
        }
        if (stacks) {
            require(stacks->plan == plan, "the stack set belongs to another plan");
            swap_binding(n, *plan, *stacks);
            n.bound = stacks;
        }
    });
}

int cpde_stacks_destroy(cpde_stacks* stacks) {
    return guarded([&] {
        if (!stacks) return;
        Net& n = *stacks->plan->net;
        sync_stream(*n.dev, __LINE__);
        if (n.bound == stacks) {
            swap_binding(n, *stacks->plan, *stacks);
            n.bound = nullptr;
        }
        ++n.dev->layout;
        for (auto* v : {&stacks->z, &stacks->y, &stacks->g})
            for (float* q : *v) (void)hipFree(q);
        (void)hipFree(stacks->input);
        delete stacks;
    });
}

int cpde_plan_stack(cpde_plan* plan, int layer, int kind, float** device_ptr) {
    return guarded([&] {
        Net& n = *plan->net;
        require(layer >= 0 && layer < n.layers && kind >= 0 && kind <= 3, "invalid stack");
        // network-fused plans keep u (the jet of sigma'(z)) where the others keep z
        const bool keeps_u = plan->fused && plan->network && !n.linear[layer];
        require(!(kind == 0 && keeps_u), "this plan keeps u, not z, for a sigmoid layer (stack kind 3)");
        require(!(kind == 3 && !keeps_u), "u is kept only by network-fused plans for sigmoid layers");
        float* p = kind == 0 || kind == 3 ? (layer == 0 ? plan->input : n.z[layer]) : kind == 1 ? n.y[layer] : n.g[layer];
        require(p != nullptr, "stack not present for this layer");
        *device_ptr = p;
    });
}

int cpde_plan_stack_scale(cpde_plan* plan, int layer, int kind, float* row_factor) {
    return guarded([&] {
        Net& n = *plan->net;
        require(layer >= 0 && layer < n.layers && kind >= 0 && kind <= 3 && row_factor, "invalid stack");
        // scaled network kernels: sigmoid layers hold y, u as row / alpha! and dE/dz as alpha! dE/dz
        const bool scaled = plan->fused && plan->network && plan->fused->scaled && !n.linear[layer] && kind != 0;
        for (int r = 0; r < plan->rows; ++r) {
            double f = 1.0;
            for (int v = 0; v < plan->tables.variables; ++v)
                for (int k = 2; k <= plan->tables.table[r * (plan->tables.variables + 1) + 1 + v]; ++k) f *= k;
            row_factor[r] = !scaled ? 1.0f : kind == 2 ? float(1.0 / f) : float(f);
        }
    });
}

// ---- hot path ------------------------------------------------------------------------------
int cpde_activate(cpde_plan* plan, const float* data, int data_width, const int* rows, int offset, int valid) {
    return guarded([&] {
        flush_wgrad(*plan->net->dev);  // this call writes stacks a waiting launch may read
        Net& n = *plan->net;
        Device& d = *n.dev;
        require(valid >= 0 && valid <= plan->width && offset >= 0 && offset + valid <= data_width,
                "invalid chunk range");
        reserve_arena(n, *plan);
        launch_activate(d, plan->input, data, data_width, n.neurons[0], plan_rows(*plan, rows), plan->rows, plan->width,
                        offset, valid);
    });
}

int cpde_forward(cpde_plan* plan) {
    return guarded([&] {
        flush_wgrad(*plan->net->dev);  // this call writes stacks a waiting launch may read
        Net& n = *plan->net;
        Device& d = *n.dev;
        if (plan->fused) {
            fused_forward(*plan);
            return;
        }
        const int cols = int(plan->columns());
        for (int t = 0; t + 1 < n.layers; ++t) {
            const int ni = n.neurons[t], no = n.neurons[t + 1];
            if (!n.linear[t]) launch_compose_forward(d, *plan, n.z[t], n.y[t], ni);
            const float* W = n.state[0][t];
            launch_gemm(d, no, cols, ni, W, no, false, activations(*plan, t), ni, false, n.z[t + 1], no,
                        W + size_t(no) * ni, plan->rows);
        }
    });
}

int cpde_output(cpde_plan* plan, float* dest, int dest_width, const int* rows, int offset, int valid) {
    return guarded([&] {
        Net& n = *plan->net;
        Device& d = *n.dev;
        require(valid >= 0 && valid <= plan->width && offset + valid <= dest_width, "invalid chunk range");
        flush_wgrad(d);  // the outputs of a held epoch
        launch_output(d, dest, n.z[n.layers - 1], dest_width, n.neurons.back(), plan_rows(*plan, rows), plan->rows,
                      plan->width, offset, valid);
    });
}

int cpde_costs_begin(cpde_device* dev, int costs) {
    return guarded([&] {
        flush_reduce(*dev);
        launch_costs_begin(*dev, costs);
    });
}

int cpde_gradients_defer(cpde_device* dev, int on) {
    return guarded([&] {
        require(dev, "null argument");
        dev->defer = on != 0;
        if (!on) flush_reduce(*dev);
    });
}

int cpde_cost_matching(cpde_plan* plan, const float* target, int target_width, const int* target_rows,
                       const float* weights, int weight_samples, int offset, int valid, int cost_index, int collect,
                       int gradient) {
    return guarded([&] {
        flush_wgrad(*plan->net->dev);  // this call writes stacks a waiting launch may read
        flush_if_reads(*plan->net->dev, nullptr, cost_index);
        Net& n = *plan->net;
        Device& d = *n.dev;
        require(cost_index >= 0 && cost_index < d.cost_capacity, "cost slot out of range");
        require(!gradient || plan->backward, "plan has no adjoint storage");
        const int L = n.layers;
        launch_matching(d, *plan, n.z[L - 1], gradient ? n.g[L - 1] : nullptr, target, target_width, target_rows,
                        weights, weight_samples, offset, valid, cost_index, collect != 0, gradient != 0);
    });
}

int cpde_epoch_matching(cpde_plan* plan, const float* target, int target_width, const int* target_rows,
                        const float* weights, int weight_samples, int offset, int valid, int cost_index, int collect,
                        int accumulate) {
    return guarded([&] {
        Net& n = *plan->net;
        Device& d = *n.dev;
        require(cost_index >= 0 && cost_index < d.cost_capacity, "cost slot out of range");
        require(plan->backward, "plan has no adjoint storage");
        require(valid >= 0 && valid <= plan->width && offset >= 0, "invalid chunk range");
        if (!one_pass_fits(*plan)) {
            if (int code = cpde_forward(plan)) throw_code(code);
            if (int code = cpde_cost_matching(plan, target, target_width, target_rows, weights, weight_samples, offset,
                                              valid, cost_index, collect, 1))
                throw_code(code);
            if (int code = cpde_backward(plan, accumulate)) throw_code(code);
            return;
        }
        CostStats* records = epoch_records(*plan);
        MatchArgsHost m{target, target_rows, weights, records, target_width, weight_samples, offset, valid,
                        collect != 0};
        one_pass_epoch(*plan, plan->fused->network_epoch, &m, records, cost_index, accumulate != 0);
    });
}

int cpde_epoch_matching_rprop(cpde_plan* plan, const float* target, int target_width, const int* target_rows,
                              const float* weights, int weight_samples, int offset, int valid, int cost_index,
                              int collect, int accumulate) {
    return guarded([&] {
        Net& n = *plan->net;
        Device& d = *n.dev;
        require(cost_index >= 0 && cost_index < d.cost_capacity, "cost slot out of range");
        require(plan->backward, "plan has no adjoint storage");
        require(valid >= 0 && valid <= plan->width && offset >= 0, "invalid chunk range");
        if (!one_pass_fits(*plan) || n.layers - 1 > kMaxTransitions) {
            if (int code = cpde_epoch_matching(plan, target, target_width, target_rows, weights, weight_samples, offset,
                                               valid, cost_index, collect, accumulate))
                throw_code(code);
            launch_rprop(d, n);
            return;
        }
        CostStats* records = epoch_records(*plan);
        MatchArgsHost m{target, target_rows, weights, records, target_width, weight_samples, offset, valid,
                        collect != 0};
        one_pass_epoch(*plan, plan->fused->network_epoch, &m, records, cost_index, accumulate != 0, {}, true);
    });
}

int cpde_epoch_matching_static(cpde_plan* plan, const float* target, int target_width, const int* target_rows,
                               const float* weights, int weight_samples, int offset, int valid, int cost_index,
                               int collect, int accumulate) {
    return guarded([&] {
        flush_reduce(*plan->net->dev);
        Net& n = *plan->net;
        Device& d = *n.dev;
        if (!d.static_scratch) throw invalid("no static scratch on this device: " + d.static_scratch_error);
        require(!d.tracing, "kernel tracing records events: the no-allocation epoch runs with tracing off");
        require(cost_index >= 0 && cost_index < d.cost_capacity, "cost slot out of range");
        require(plan->backward, "plan has no adjoint storage");
        require(valid >= 0 && valid <= plan->width && offset >= 0, "invalid chunk range");
        require(one_pass_fits(*plan),
                "the no-allocation epoch needs a plan whose one-pass epoch applies (network-fused kernels, the "
                "chunk's workgroups resident on the device together)");
        const int blocks = epoch_blocks(*plan);
        const size_t record_bytes = (sizeof(CostStats) * size_t(blocks) + 255) / 256 * 256;
        require(record_bytes < size_t(CPDE_STATIC_SCRATCH_BYTES), "cost records beyond the static scratch");
        CostStats* records = reinterpret_cast<CostStats*>(d.static_scratch);
        const PartialSpace space{reinterpret_cast<float*>(d.static_scratch + record_bytes),
                                 (size_t(CPDE_STATIC_SCRATCH_BYTES) - record_bytes) / sizeof(float)};
        MatchArgsHost m{target, target_rows, weights, records, target_width, weight_samples, offset, valid,
                        collect != 0};
        one_pass_epoch(*plan, plan->fused->network_epoch, &m, records, cost_index, accumulate != 0, space);
    });
}

int cpde_cost_polynomial(cpde_plan* plan, const cpde_poly_term* terms, int term_count, const float* coefficients,
                         const float* rhs, const float* weights, int equations, int samples, int offset, int valid,
                         int cost_index, int collect, int gradient) {
    return guarded([&] {
        flush_wgrad(*plan->net->dev);  // this call writes stacks a waiting launch may read
        flush_if_reads(*plan->net->dev, nullptr, cost_index);
        Net& n = *plan->net;
        Device& d = *n.dev;
        require(cost_index >= 0 && cost_index < d.cost_capacity, "cost slot out of range");
        require(!gradient || plan->backward, "plan has no adjoint storage");
        const int L = n.layers;
        launch_polynomial(d, *plan, n.z[L - 1], gradient ? n.g[L - 1] : nullptr, terms, term_count, coefficients, rhs,
                          weights, equations, samples, offset, valid, cost_index, collect != 0, gradient != 0);
    });
}

int cpde_scale_adjoint(cpde_plan* plan, const double* multiplier) {
    return guarded([&] {
        flush_wgrad(*plan->net->dev);  // this call writes stacks a waiting launch may read
        Net& n = *plan->net;
        launch_scale_adjoint(*n.dev, *plan, n.g[n.layers - 1], multiplier);
    });
}

int cpde_backward(cpde_plan* plan, int accumulate) {
    return guarded([&] {
        flush_wgrad(*plan->net->dev);  // this call writes stacks a waiting launch may read
        Net& n = *plan->net;
        Device& d = *n.dev;
        require(plan->backward, "plan has no adjoint storage");
        if (plan->fused) {
            fused_backward(*plan, accumulate != 0);
            return;
        }
        // dE/dz of every layer (transposed products, in-place adjoint
        // compositions), then all weight gradients in one grouped launch
        const int cols = int(plan->columns());
        for (int t = n.layers - 2; t >= 1; --t) {
            const int ni = n.neurons[t], no = n.neurons[t + 1];
            launch_gemm(d, ni, cols, no, n.state[0][t], no, true, n.g[t + 1], no, false, n.g[t], ni, nullptr, 1);
            if (!n.linear[t]) launch_compose_adjoint(d, *plan, n.z[t], n.g[t], ni);
        }
        weight_gradients(*plan, accumulate != 0);
    });
}

// ---- reductions and optimizers --------------------------------------------------------------
int cpde_inspect_gradients(cpde_net* net) {
    return guarded([&] {
        flush_reduce(*net->dev);
        Device& d = *net->dev;
        const int T = net->layers - 1;
        d.reserve_grads(T);
        for (int first = 0; first < T; first += kMaxTransitions) {
            const int n = std::min(kMaxTransitions, T - first);
            const float* g[kMaxTransitions];
            int counts[kMaxTransitions];
            for (int k = 0; k < n; ++k) {
                g[k] = net->state[net->active[first + k]][first + k];
                counts[k] = net->param_count(first + k);
            }
            launch_grad_stats(d, g, counts, n, first);
        }
    });
}

int cpde_scalars_download(cpde_device* dev, int costs, cpde_cost_stats* cost_out, int layers,
                          cpde_gradient_stats* gradient_out) {
    return cpde_scalars_download_graph(dev, costs, cost_out, layers, gradient_out, nullptr, nullptr);
}

int cpde_scalars_download_graph(cpde_device* dev, int costs, cpde_cost_stats* cost_out, int layers,
                                cpde_gradient_stats* gradient_out, const cpde_graph_summary* summary,
                                cpde_graph_summary* summary_out) {
    return guarded([&] {
        flush_reduce(*dev);
        require(costs <= dev->cost_capacity && layers <= dev->grad_capacity, "scalar slots out of range");
        require(summary == nullptr || summary_out != nullptr, "graph summary without a destination");
        const bool own_summary = summary == nullptr && summary_out != nullptr;
        if (own_summary) {  // one copy over the whole block: costs, gradient totals and the summary slot
            HIP_CHECK(hipMemcpyAsync(dev->host_block, dev->scalar_block, dev->scalar_bytes, hipMemcpyDeviceToHost,
                                     dev->stream));
        } else if (costs && layers) {  // one copy over both (the block keeps them in this order)
            const size_t bytes = size_t(reinterpret_cast<char*>(dev->grad_totals + layers) -
                                        static_cast<char*>(dev->scalar_block));
            HIP_CHECK(hipMemcpyAsync(dev->host_block, dev->scalar_block, bytes, hipMemcpyDeviceToHost, dev->stream));
        } else if (costs) {
            HIP_CHECK(hipMemcpyAsync(dev->host_costs, dev->cost_totals, sizeof(CostStats) * costs,
                                     hipMemcpyDeviceToHost, dev->stream));
        } else if (layers) {
            HIP_CHECK(hipMemcpyAsync(dev->host_grads, dev->grad_totals, sizeof(GradStats) * layers,
                                     hipMemcpyDeviceToHost, dev->stream));
        }
        if (summary)
            HIP_CHECK(hipMemcpyAsync(dev->host_summary, summary, sizeof(cpde_graph_summary), hipMemcpyDeviceToHost,
                                     dev->stream));
        sync_stream(*dev, __LINE__);
        if (costs && cost_out) {
            std::memcpy(cost_out, dev->host_costs, sizeof(CostStats) * costs);
            for (int i = 0; i < costs && i < int(dev->slot_fresh.size()); ++i)
                if (dev->slot_fresh[i]) cost_out[i] = cpde_cost_stats{0.0, INT32_MAX, INT32_MAX};
        }
        if (layers && gradient_out) std::memcpy(gradient_out, dev->host_grads, sizeof(GradStats) * layers);
        if (summary) *summary_out = *dev->host_summary;
        if (own_summary) *summary_out = *dev->host_graph_summary;
    });
}

// cpde_update_issue; with `inspect`, cpde_inspect_gradients first -- or, where
// the statistics need not be whole (`full` false) and update_tests(net) holds,
// the update launch's own finiteness test in their place.
static int issue_update(cpde_device* dev, int costs, int layers, int with_graph, cpde_net* net, int method, int step,
                        float lr, bool inspect, bool full) {
    return guarded([&] {
        require(dev && net, "null argument");
        bool test = false;
        if (inspect) {
            if (full || !update_tests(*net)) {
                if (int code = cpde_inspect_gradients(net)) throw_code(code);
            } else {
                test = true;
                flush_reduce(*dev);
                dev->reserve_grads(net->layers - 1);
            }
        }
        require(method == 0 || (method == 1 && step >= 1), "method 0 (RPROP) or 1 (Adam, step >= 1)");
        require(net->dev == dev, "network of another device");
        require(!dev->issued.open, "an issued update is not resolved yet");
        require(costs >= 0 && costs <= 64, "at most 64 cost slots");
        require(costs <= dev->cost_capacity && layers == net->layers - 1 && layers <= dev->grad_capacity,
                "scalar slots out of range");
        flush_reduce(*dev);
        // one copy over costs, gradient totals and (with a graph) the summary
        // slot, made by the update launch's first workgroup (no copy launch of
        // its own); the host waits for that launch
        const size_t bytes = with_graph ? dev->scalar_bytes
                                        : size_t(reinterpret_cast<char*>(dev->grad_totals + layers) -
                                                 static_cast<char*>(dev->scalar_block));
        const ScalarPublish copy{dev->scalar_block, dev->host_block, bytes};
        unsigned long long fresh = 0;
        for (int i = 0; i < costs && i < int(dev->slot_fresh.size()); ++i)
            if (dev->slot_fresh[i]) fresh |= 1ull << i;
        // with its own test the launch reads no gradient totals
        const UpdateGuard guard{dev->cost_totals, costs, fresh, test ? nullptr : dev->grad_totals, test ? 0 : layers,
                                with_graph ? dev->graph_summary : nullptr};
        const bool wt_current = net->wt_current;
        if (method == 0) {
            launch_rprop(*dev, *net, &guard, &copy, test);
            rprop_done(*net);  // in expectation; cpde_update_resolve switches back if the rule rejects the epoch
        } else {
            launch_adam(*dev, *net, step, lr, &guard, &copy, test);
        }
        HIP_CHECK(hipEventRecord(dev->copied, dev->stream));
        dev->issued = Device::IssuedUpdate{true, net, costs, layers, with_graph != 0, method == 0, wt_current, fresh};
    });
}

int cpde_update_issue(cpde_device* dev, int costs, int layers, int with_graph, cpde_net* net, int method, int step,
                      float lr) {
    return issue_update(dev, costs, layers, with_graph, net, method, step, lr, false, false);
}

int cpde_inspect_update_issue(cpde_device* dev, int costs, int layers, int with_graph, cpde_net* net, int method,
                              int step, float lr, int full_stats) {
    return issue_update(dev, costs, layers, with_graph, net, method, step, lr, true, full_stats != 0);
}

int cpde_update_resolve(cpde_device* dev, cpde_cost_stats* cost_out, cpde_gradient_stats* gradient_out,
                        cpde_graph_summary* summary_out, int* updated) {
    return guarded([&] {
        require(dev && updated, "null argument");
        require(dev->issued.open, "no issued update");
        Device::IssuedUpdate u = dev->issued;
        dev->issued.open = false;
        HIP_CHECK(hipEventSynchronize(dev->copied));
        if (u.costs && cost_out) {
            std::memcpy(cost_out, dev->host_costs, sizeof(CostStats) * u.costs);
            for (int i = 0; i < u.costs; ++i)
                if ((u.fresh >> i) & 1ull) cost_out[i] = cpde_cost_stats{0.0, INT32_MAX, INT32_MAX};
        }
        if (gradient_out) std::memcpy(gradient_out, dev->host_grads, sizeof(GradStats) * u.layers);
        if (u.graph && summary_out) *summary_out = *dev->host_graph_summary;
        // the rule on the bytes the kernel read
        const UpdateGuard guard{dev->host_costs, u.costs, u.fresh, dev->host_grads, u.layers,
                                u.graph ? dev->host_graph_summary : nullptr};
        *updated = update_accepted(guard) ? 1 : 0;
        if (!*updated) {  // the update did not apply: RPROP's buffers switch back
            if (u.rprop) rprop_done(*u.net);
            u.net->wt_current = u.wt_current;
        }
    });
}

int cpde_scalars_download_rprop(cpde_device* dev, int costs, cpde_cost_stats* cost_out, int layers,
                                cpde_gradient_stats* gradient_out, cpde_graph_summary* summary_out, cpde_net* net,
                                int* updated) {
    if (int code = cpde_update_issue(dev, costs, layers, summary_out ? 1 : 0, net, 0, 0, 0.0f)) return code;
    return cpde_update_resolve(dev, cost_out, gradient_out, summary_out, updated);
}

int cpde_gradients_discard(cpde_device* dev) {
    return guarded([&] {
        require(dev, "null argument");
        if (dev->held) dev->held->open = false;
        dev->waiting = Device::PendingReduce{};
        dev->defer = false;
    });
}

int cpde_rprop(cpde_net* net) {
    return guarded([&] {
        flush_reduce(*net->dev);
        launch_rprop(*net->dev, *net);
    });
}

int cpde_adam(cpde_net* net, int step, float lr) {
    return guarded([&] {
        flush_reduce(*net->dev);
        require(step >= 1, "Adam step must be positive");
        launch_adam(*net->dev, *net, step, lr);
    });
}

int cpde_set_steps(cpde_net* net, float value) {
    return guarded([&] {
        flush_reduce(*net->dev);
        launch_set_steps(*net->dev, *net, value);
    });
}

int cpde_restore_steps(cpde_net* net, float floor_value) {
    return guarded([&] {
        flush_reduce(*net->dev);
        launch_restore_steps(*net->dev, *net, floor_value);
    });
}

int cpde_zero_gradient(cpde_net* net) {
    return guarded([&] {
        flush_reduce(*net->dev);
        std::vector<float*> p;
        std::vector<int> counts;
        for (int t = 0; t + 1 < net->layers; ++t) {
            p.push_back(net->state[net->active[t]][t]);
            counts.push_back(net->param_count(t));
        }
        launch_fill_grouped(*net->dev, p.data(), counts.data(), int(p.size()), 0.0f);
    });
}

int cpde_reset_optimizer(cpde_net* net) {
    return guarded([&] {
        flush_reduce(*net->dev);
        for (int t = 0; t + 1 < net->layers; ++t) {
            net->active[t] = 1;
            for (int b = 1; b < 4; ++b) launch_fill(*net->dev, net->state[b][t], net->param_count(t), 0.0f);
        }
    });
}

// ---- expression programs (hipRTC) ----------------------------------------------------------
int cpde_program_compile(cpde_device* dev, const char* source, cpde_program** out, char* log, size_t log_capacity) {
    return guarded([&] {
        require(source && out, "null argument");
        static std::atomic<uint64_t> next_id{1};
        std::string text;
        std::vector<char> code;
        try {
            code = compile_module(source, device_arch(dev->ordinal), &text);
        } catch (const compile_error&) {
            if (log && log_capacity) std::snprintf(log, log_capacity, "%s", text.c_str());
            throw compile_error("expression compile failed: " + text);
        }
        if (log && log_capacity) std::snprintf(log, log_capacity, "%s", text.c_str());
        auto p = std::make_unique<cpde_program>();
        p->dev = dev;
        p->log = text;
        p->source = source;
        p->id = next_id++;
        HIP_CHECK(hipModuleLoadData(&p->module, code.data()));
        HIP_CHECK(hipModuleGetFunction(&p->function, p->module, "expression"));
        *out = p.release();
    });
}

int cpde_program_destroy(cpde_program* program) {
    return guarded([&] {
        if (!program) return;
        sync_stream(*program->dev, __LINE__);
        ++program->dev->layout;
        if (program->module) (void)hipModuleUnload(program->module);
        delete program;
    });
}

int cpde_cost_expression(cpde_plan* plan, cpde_program* program, const double* fields,
                         const double* quadrature_weights, int samples, int offset, int valid,
                         const double* multiplier, void* scratch, int cost_index, int collect, int gradient) {
    return guarded([&] {
        flush_wgrad(*plan->net->dev);  // this call writes stacks a waiting launch may read
        flush_if_reads(*plan->net->dev, nullptr, cost_index);
        Net& n = *plan->net;
        Device& d = *n.dev;
        require(cost_index >= 0 && cost_index < d.cost_capacity, "cost slot out of range");
        require(!gradient || plan->backward, "plan has no adjoint storage");
        const float* y = n.z[n.layers - 1];
        float* g = gradient ? n.g[n.layers - 1] : nullptr;
        double* loss = static_cast<double*>(scratch);
        int* bad = reinterpret_cast<int*>(loss + plan->width);
        int outputs = n.neurons.back(), rows = plan->rows, width = plan->width;
        int col = collect, grd = gradient;
        void* args[] = {&y, &g, &fields, &quadrature_weights, &loss, &bad, &outputs, &rows, &samples, &width,
                        &offset, &valid, &multiplier, &col, &grd};
        const int blocks = std::max(1, std::min(kMaxCostBlocks, (width + kCostThreads - 1) / kCostThreads));
        HIP_CHECK(hipModuleLaunchKernel(program->function, blocks, 1, 1, kCostThreads, 1, 1, 0, d.stream, args,
                                        nullptr));
        launch_sample_reduce(d, loss, bad, valid, offset, cost_index);
    });
}

// Whether a program's source defines the per-sample functions that the one-pass
// expression epoch compiles into the network module (the input gather and the
// point function).
static bool defines_point_function(const cpde_program& program) {
    return program.source.find("cpde_expression_point") != std::string::npos &&
           program.source.find("cpde_expression_inputs") != std::string::npos;
}

int cpde_epoch_expression(cpde_plan* plan, cpde_program* program, const double* fields,
                          const double* quadrature_weights, int samples, int offset, int valid, const double* multiplier,
                          void* scratch, int cost_index, int collect, int accumulate) {
    return guarded([&] {
        Net& n = *plan->net;
        Device& d = *n.dev;
        require(program, "null argument");
        require(cost_index >= 0 && cost_index < d.cost_capacity, "cost slot out of range");
        require(plan->backward, "plan has no adjoint storage");
        require(valid >= 0 && valid <= plan->width && offset >= 0, "invalid chunk range");
        const bool one_pass =
            one_pass_fits(*plan) && defines_point_function(*program);
        if (!one_pass) {
            if (int code = cpde_forward(plan)) throw_code(code);
            if (int code = cpde_cost_expression(plan, program, fields, quadrature_weights, samples, offset, valid,
                                                multiplier, scratch, cost_index, collect, 1))
                throw_code(code);
            if (int code = cpde_backward(plan, accumulate)) throw_code(code);
            return;
        }
        const hipFunction_t kernel = expression_epoch(*plan, *program);
        CostStats* records = epoch_records(*plan);
        ExpressionArgsHost e{fields, quadrature_weights, multiplier, records, samples, offset, valid, collect != 0};
        one_pass_epoch(*plan, kernel, &e, records, cost_index, accumulate != 0, {}, false, program);
    });
}

int cpde_epoch_expression_fused(cpde_plan* plan, cpde_program* program, int* fused) {
    return guarded([&] {
        require(plan && program && fused, "null argument");
        *fused = plan->backward && one_pass_fits(*plan) &&
                 defines_point_function(*program);
    });
}

int cpde_graph_execute(cpde_device* dev, const cpde_scalar_node* nodes, int count, int root, int leaves,
                       double* values, double* adjoints, double* multipliers, int* active, cpde_graph_summary* summary,
                       int gradient) {
    return guarded([&] {
        require(leaves <= dev->cost_capacity, "graph leaves exceed cost slots");
        const GraphLaunch g = graph_launch(*dev, nodes, count, root, leaves, values, adjoints, multipliers, active,
                                           summary ? summary : dev->graph_summary, gradient != 0);
        launch_clear_fresh(*dev, leaves);
        Device::PendingReduce& w = dev->waiting;
        if (w.open && !w.ra.with_graph) {
            // the graph rides in the waiting reduction, after its cost finishes
            w.ra.with_graph = 1;
            w.ra.graph = g;
            flush_reduce(*dev);
        } else {
            flush_reduce(*dev);
            launch_graph(*dev, g);
        }
    });
}

int cpde_trace_enable(cpde_device* dev, int on) {
    return guarded([&] {
        flush_reduce(*dev);
        require(!dev->capturing, "a capture is open on this device");
        dev->fold_trace();
        dev->tracing = on != 0;
        for (int k = 0; k < kTraceKinds; ++k) {
            dev->trace_ms[k] = dev->trace_work[k] = 0;
            dev->trace_launches[k] = 0;
        }
    });
}

int cpde_trace_read(cpde_device* dev, int kind, uint64_t* launches, double* total_ms, double* work) {
    return guarded([&] {
        flush_reduce(*dev);
        require(kind >= 0 && kind < kTraceKinds, "invalid trace kind");
        dev->fold_trace();
        if (launches) *launches = dev->trace_launches[kind];
        if (total_ms) *total_ms = dev->trace_ms[kind];
        if (work) *work = dev->trace_work[kind];
    });
}

const char* cpde_trace_name(int kind) {
    static const char* names[kTraceKinds] = {
        "compose_forward", "compose_adjoint", "gemm_forward",   "gemm_transposed", "gemm_wgrad",
        "split_reduce",    "bias_grad",       "activate",       "cost",            "reduce",
        "optimizer",       "other",           "fused_input",    "fused_forward",   "fused_backward",
        "fused_output_backward", "network_forward", "network_backward", "network_epoch"};
    return kind >= 0 && kind < kTraceKinds ? names[kind] : "";
}

int cpde_trace_kinds(void) { return kTraceKinds; }

int cpde_jit_prepare(int rows, int variables, const int* table, int layers, const int* neurons, int width,
                     int compute_units, const char* arch, char* log, size_t log_capacity) {
    return guarded([&] {
        require(table && neurons && arch && layers >= 3, "invalid argument");
        const Tables t = build_tables(rows, variables, table);
        std::string text;
        try {
            const std::vector<int> n(neurons, neurons + layers);
            compile_module(fused_source(t, n, tuning(t.rows, width, compute_units, n)), arch, &text);
        } catch (...) {
            if (log && log_capacity) std::snprintf(log, log_capacity, "%s", text.c_str());
            throw;
        }
        if (log && log_capacity) std::snprintf(log, log_capacity, "%s", text.c_str());
    });
}

int cpde_mark(cpde_device* dev, int slot) {
    return guarded([&] {
        flush_reduce(*dev);
        require(slot >= 0 && slot < 8, "invalid event slot");
        require(!dev->capturing, "a capture is open on this device");
        HIP_CHECK(hipEventRecord(dev->marks[slot], dev->stream));
    });
}

int cpde_elapsed(cpde_device* dev, int from_slot, int to_slot, float* ms) {
    return guarded([&] {
        require(from_slot >= 0 && from_slot < 8 && to_slot >= 0 && to_slot < 8, "invalid event slot");
        HIP_CHECK(hipEventSynchronize(dev->marks[to_slot]));
        HIP_CHECK(hipEventElapsedTime(ms, dev->marks[from_slot], dev->marks[to_slot]));
    });
}

// ---- captured epochs --------------------------------------------------------------------
int cpde_capture_begin(cpde_device* dev) {
    return guarded([&] {
        require(dev, "null argument");
        require(!dev->capturing, "a capture is already open on this device");
        require(!dev->tracing, "tracing times every launch with events; a capture cannot hold them");
        flush_reduce(*dev);
        dev->capture_nets.clear();
        for (Net* n : dev->nets) dev->capture_nets.push_back({n, n->active});
        dev->capture_layout = dev->layout;
        HIP_CHECK(hipStreamBeginCapture(dev->stream, hipStreamCaptureModeThreadLocal));
        dev->capturing = true;
    });
}

// The recorded calls never ran: their host bookkeeping is undone (active
// gradient buffers back to the capture's start; the row-major weight copies
// are rewritten before their next use).
static void abandon_capture(Device& d) {
    for (auto& c : d.capture_nets) {
        c.net->active = c.active;
        c.net->wt_current = false;
    }
    d.capture_nets.clear();
}

int cpde_capture_end(cpde_device* dev, int keep, cpde_replay** out) {
    return guarded([&] {
        require(dev, "null argument");
        if (out) *out = nullptr;
        require(dev->capturing, "no capture is open on this device");
        flush_reduce(*dev);  // recorded with the rest
        dev->capturing = false;
        hipGraph_t graph = nullptr;
        const hipError_t ended = hipStreamEndCapture(dev->stream, &graph);
        const bool intact = dev->layout == dev->capture_layout;
        hipGraphExec_t exec = nullptr;
        hipError_t made = hipSuccess;
        if (keep && out && ended == hipSuccess && graph && intact)
            made = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (graph) (void)hipGraphDestroy(graph);
        if (!exec) {
            abandon_capture(*dev);
            if (!keep) return;
            require(out != nullptr, "null output");
            HIP_CHECK(ended);
            HIP_CHECK(made);
            require(intact, "device memory was released or regrown during the capture");
            throw invalid("the capture recorded nothing");
        }
        auto r = std::make_unique<cpde_replay>();
        r->dev = dev;
        r->exec = exec;
        r->layout = dev->layout;
        for (auto& c : dev->capture_nets) r->nets.push_back({c.net, c.active, c.net->active, c.net->generation});
        dev->capture_nets.clear();
        // the recorded calls have done their host bookkeeping: their device
        // work runs now
        const hipError_t launched = hipGraphLaunch(exec, dev->stream);
        if (launched != hipSuccess) {
            (void)hipGraphExecDestroy(exec);
            for (auto& c : r->nets) {
                c.net->active = c.before;
                c.net->wt_current = false;
            }
            HIP_CHECK(launched);
        }
        *out = r.release();
    });
}

int cpde_replay_launch(cpde_replay* replay) {
    return guarded([&] {
        require(replay, "null argument");
        Device& d = *replay->dev;
        require(!d.capturing, "a capture is open on this device");
        require(d.layout == replay->layout, "device memory was released or regrown since the capture");
        for (const auto& c : replay->nets) {
            require(c.net->active == c.before, "a network's active gradient buffers differ from the capture's");
            require(c.net->generation == c.generation, "a network's stack arena changed since the capture");
        }
        flush_reduce(d);
        for (const auto& c : replay->nets)
            if (!c.net->wt_current) refresh_wt(*c.net);
        HIP_CHECK(hipGraphLaunch(replay->exec, d.stream));
        for (const auto& c : replay->nets) c.net->active = c.after;
    });
}

int cpde_replay_destroy(cpde_replay* replay) {
    return guarded([&] {
        if (!replay) return;
        sync_stream(*replay->dev, __LINE__);
        (void)hipGraphExecDestroy(replay->exec);
        delete replay;
    });
}

}  // extern "C"
