// Internal declarations shared by the device library's translation units.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/cpde_hip.h"

namespace cpde {

// Raised for invalid arguments; the C ABI maps it to CPDE_EINVAL.
struct invalid : std::runtime_error {
    using std::runtime_error::runtime_error;
};
// Raised for HIP runtime failures; mapped to CPDE_EDEVICE.
struct device_error : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct compile_error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void set_error(const std::string& message);
void check_hip(hipError_t status, const char* what, const char* file, int line);
#define HIP_CHECK(expr) ::cpde::check_hip((expr), #expr, __FILE__, __LINE__)
inline void require(bool ok, const char* message) {
    if (!ok) throw invalid(message);
}

constexpr int kMaxOrder = 6;
constexpr int kMaxRows = 255;      // row indices are stored in 8 bits in the term tables
constexpr int kMaxTransitions = 32;  // per fused optimizer launch
constexpr int kCostThreads = 256;
constexpr int kMaxCostBlocks = 1024;
constexpr int kWgradChunk = 32;         // columns per LDS chunk of the weight-gradient tiles
constexpr int kWgradMinColumns = 1024;  // shorter 128x128 splits switch to 64x64 tiles

// Device-side mirrors of the public reduction structs.
struct CostStats {
    double value;
    int bad_sample, bad_component;
};
struct GradStats {
    double squared_norm, max_abs;
    unsigned long long nonfinite;
    int first, pad_;
};
// Whether a training epoch's update is accepted -- the rule the protocol
// server applies before it updates (cuda/cpde_server.cu:394-410): every cost
// finite and without a bad sample (the slots in the `fresh` mask, not written
// this epoch, count as clean), the graph, if any, without a bad node, every
// gradient finite.  One rule for the host and the device, so that an update
// launched before the host has looked decides as the host will.
struct UpdateGuard {
    const CostStats* costs = nullptr;
    int cost_count = 0;
    unsigned long long fresh = 0;
    const GradStats* grads = nullptr;
    int grad_count = 0;
    const cpde_graph_summary* graph = nullptr;
};
__host__ __device__ inline bool update_accepted(const UpdateGuard& g) {
    for (int c = 0; c < g.cost_count; ++c) {
        if ((g.fresh >> c) & 1ull) continue;
        if (g.costs[c].bad_sample != 0x7fffffff || !__builtin_isfinite(g.costs[c].value)) return false;
    }
    if (g.graph && g.graph->bad_node >= 0) return false;
    for (int t = 0; t < g.grad_count; ++t)
        if (g.grads[t].nonfinite != 0) return false;
    return true;
}
static_assert(sizeof(CostStats) == sizeof(cpde_cost_stats), "cost stats layout");
static_assert(sizeof(GradStats) == sizeof(cpde_gradient_stats), "gradient stats layout");

// Composition term tables for one schema (built on the host, see tables.cpp).
//   forward:   for row r >= 1 at fwd_offset[r]: order k, then for m = 1..k a count
//              c_m followed by c_m records {coefficient bits, packed block rows};
//              block rows are 8-bit, packed little-endian into two ints.
//   adjoint:   for row i at pair_offset[i]: count, then records {j, dn, coefficient}.
struct Tables {
    int rows = 0, variables = 0;
    std::vector<int> table;        // rows x (variables+1)
    std::vector<int> words;        // forward section then adjoint section
    std::vector<int> fwd_offset;   // per row
    std::vector<int> pair_offset;  // per row
    int forward_terms = 0, pair_terms = 0, max_order = 0;
};
Tables build_tables(int rows, int variables, const int* table);

struct Device;
struct FusedModule;
struct ExpressionEpoch;

struct Net {
    Device* dev = nullptr;
    int layers = 0;
    std::vector<int> neurons, linear;
    // Per transition t: four state buffers of n_{t+1} x (n_t+1) floats.
    std::vector<float*> state[4];
    std::vector<int> active;  // 1 or 2 per transition
    // Per transition: n_t x n_{t+1} row-major copy of the weights (without the
    // bias) for the backward's products.  Written by every network-fused
    // forward and by the optimizer launches; the one-pass epoch transposes
    // first only when wt_current is false (a new network, or the weights'
    // device pointer handed out by cpde_net_state).
    std::vector<float*> wt;
    bool wt_current = false;
    // Stack arena shared by every plan of the network (contexts are views,
    // the reference's layer banks, cuda/cpde_engine.cuh:661-693).
    std::vector<float*> z, y, g;      // per layer
    std::vector<size_t> capacity;     // floats per layer buffer
    uint64_t generation = 0;
    // split-K partial buffer for the weight-gradient contraction
    float* partials = nullptr;
    size_t partial_capacity = 0;
    size_t last_partials = 0;  // floats the previous gradient plan of the network used
    // a plan's own stack set bound in place of the arena (cpde_plan_bind); while
    // bound, the set holds the arena's pointers and the plan's own input
    struct Stacks* bound = nullptr;
    int param_count(int t) const { return neurons[t + 1] * (neurons[t] + 1); }
};

// A plan's own set of layer stacks and input chunk, for forward results kept
// until a later backward (retention): bound, it stands in for the network's
// arena and the plan's input.
struct Plan;
struct Stacks {
    Plan* plan = nullptr;
    std::vector<float*> z, y, g;
    std::vector<size_t> capacity;
    float* input = nullptr;
};

struct Plan {
    Net* net = nullptr;
    int rows = 0, variables = 0, width = 0, backward = 0;
    Tables tables;
    int* dev_tables = nullptr;  // device copy of tables.words, then tables.fwd_offset
    int* dev_rows = nullptr;    // device row map of the last activate/output
    std::vector<int> host_rows;
    // the plan's activated chunk [point][row][channel] (layer 0): its own, so
    // that plans of one network keep their inputs between epochs
    float* input = nullptr;
    std::shared_ptr<FusedModule> fused;  // null: table-driven kernels
    bool network = false;                // fused: one network-wide kernel per pass
    CostStats* epoch_partials = nullptr;  // one-pass epoch: one cost record per workgroup, two sets
    int epoch_capacity = 0, epoch_turn = 0;
    // one-pass expression epochs of this plan, by program id
    std::vector<std::pair<uint64_t, std::shared_ptr<ExpressionEpoch>>> expression_epochs;
    // layer stacks of its own, in place of the network's arena while a
    // one-pass epoch runs behind a waiting weight gradient of another plan
    // (cpde_gradients_defer); allocated on first such use
    std::vector<float*> own_z, own_y, own_g;
    uint64_t serial = 0;  // unique among the plans of the process
    // one-pass expression epochs of this plan launched together with the held
    // epoch of another plan (that plan's serial and program, this plan's program)
    struct PairedEpoch {
        uint64_t partner, partner_program, program;
        std::shared_ptr<ExpressionEpoch> epoch;
    };
    std::vector<PairedEpoch> paired_epochs;
    size_t columns() const { return size_t(rows) * size_t(width); }
};

struct Program {
    Device* dev = nullptr;
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
    std::string log;
    std::string source;  // kept for the one-pass epoch, which compiles it into the network module
    uint64_t id = 0;     // unique per compiled program
};

// Grouped weight-gradient launch (one entry per transition).
struct WgradArgs {
    const float* G[kMaxTransitions];
    const float* Y[kMaxTransitions];
    float* partial[kMaxTransitions];
    int M[kMaxTransitions], N[kMaxTransitions], kchunk[kMaxTransitions];
    int tile[kMaxTransitions];  // 128, or 64 when both sides are at most 64
    int block_begin[kMaxTransitions + 1];
    int K[kMaxTransitions], R[kMaxTransitions];  // columns and rows per point of each entry's pass
    int transitions;
    int direct;  // 1: 64x64 tiles fed straight from global memory (wgrad_direct_kernel)
};
// The scalar cost graph's evaluation (cost_graph::execute) as one lane runs it.
struct GraphLaunch {
    const cpde_scalar_node* nodes;
    const CostStats* integrals;
    double *values, *adjoints, *multipliers;
    int* active;
    cpde_graph_summary* summary;
    int count, root, leaves, gradient;
};

constexpr int kReduceCosts = 4;  // cost finishes one reduction launch carries
struct ReduceArgs {
    const float* partial[kMaxTransitions];
    float* grad[kMaxTransitions];
    int M[kMaxTransitions], N[kMaxTransitions], splits[kMaxTransitions];
    int begin[kMaxTransitions + 1];        // first entry of each transition (bytes accounting)
    int block_begin[kMaxTransitions + 1];  // first block of each transition
    int split_minor[kMaxTransitions];      // partial layout: 0 [split][entry], 1 [entry][split]
    // a second backward pass over the same entries, in the same layout: its
    // sum is added after the first's, so one launch reduces both passes bit
    // for bit as two launches in turn (splits2 0: no second pass)
    const float* partial2[kMaxTransitions];
    int splits2[kMaxTransitions];
    int transitions, accumulate, second;
    // cost finishes riding in the launch: one more block finishes them in
    // order (each as launch_finish_cost would, from at most kMaxCostBlocks
    // records), then, with `with_graph`, evaluates the scalar graph on its
    // first lane, which wrote the finished costs
    const CostStats* cost_partials[kReduceCosts];
    CostStats* cost_total[kReduceCosts];
    int cost_count[kReduceCosts], cost_overwrite[kReduceCosts];
    int costs, with_graph;
    GraphLaunch graph;
    // non-null: the gradient stores happen only if *gate is nonzero (the
    // verdict of an update issued and not yet resolved, cpde_update_issue);
    // cost finishes and the graph run either way
    const int* gate;
};
// Per-launch device timing (HIP events on the library's stream), grouped by
// kernel class.  `work` is the launch's algorithmic work: bytes for the
// HBM-bound classes, flops for the matrix-core classes.
enum TraceKind {
    kTraceComposeForward, kTraceComposeAdjoint, kTraceGemm, kTraceGemmTransposed, kTraceWgrad, kTraceSplitReduce,
    kTraceBiasGrad, kTraceActivate, kTraceCost, kTraceReduce, kTraceOptimizer, kTraceOther, kTraceFusedInput,
    kTraceFusedForward, kTraceFusedBackward, kTraceFusedOutput, kTraceNetworkForward, kTraceNetworkBackward,
    kTraceNetworkEpoch, kTraceKinds
};
// A one-pass epoch launch held back so that the next one can share it (api.hip).
struct HeldEpoch;

struct TraceRecord {
    int kind;
    double work;
    hipEvent_t start, stop;
};

struct Device {
    int ordinal = 0;
    int compute_units = 0;
    hipStream_t stream = nullptr;
    // this GPU's copy of the library's static scratch array (api.hip), or null
    // with the reason when its address could not be taken
    unsigned char* static_scratch = nullptr;
    std::string static_scratch_error;
    // reduction workspace (cuda/reduction_kernels.cuh:101-178)
    CostStats* cost_blocks = nullptr;   // kMaxCostBlocks
    // cost and gradient totals in one device block, [cost_capacity] then
    // [grad_capacity] then the graph-summary slot, mirrored by one pinned host
    // block: one copy downloads them
    void* scalar_block = nullptr;
    void* host_block = nullptr;
    CostStats* cost_totals = nullptr;   // cost_capacity, in scalar_block
    GradStats* grad_totals = nullptr;   // grad_capacity, in scalar_block
    CostStats* host_costs = nullptr;    // in host_block
    GradStats* host_grads = nullptr;
    cpde_graph_summary* host_summary = nullptr;  // pinned: one graph summary
    // the device's own graph-summary slot, after the gradient totals in
    // scalar_block (and its mirror in host_block): one copy downloads all three
    cpde_graph_summary* graph_summary = nullptr;
    cpde_graph_summary* host_graph_summary = nullptr;
    size_t scalar_bytes = 0;
    int cost_capacity = 0, grad_capacity = 0;
    hipEvent_t marks[8] = {};
    hipEvent_t copied = nullptr;  // the scalar download of an issued update
    // the guarded update's verdict (1 applied, 0 not), written by its kernel
    int* update_verdict = nullptr;
    // An update issued (cpde_update_issue) and not yet resolved: the copied
    // scalars' layout, and the network whose buffers switched in expectation.
    struct IssuedUpdate {
        bool open = false;
        Net* net = nullptr;
        int costs = 0, layers = 0;
        bool graph = false;
        bool rprop = true;        // RPROP (buffers switched in expectation), else Adam
        bool wt_current = false;  // the network's before the issue
        unsigned long long fresh = 0;
    } issued;
    // tracing
    bool tracing = false;
    std::vector<hipEvent_t> event_pool;
    std::vector<TraceRecord> pending;
    double trace_ms[kTraceKinds] = {}, trace_work[kTraceKinds] = {};
    uint64_t trace_launches[kTraceKinds] = {};
    void fold_trace();
    // fused modules compiled on this device, by source text
    std::vector<std::pair<std::string, std::shared_ptr<FusedModule>>> fused_modules;
    std::vector<std::pair<std::string, std::shared_ptr<ExpressionEpoch>>> expression_epochs;
    // Cost slots cleared by cpde_costs_begin and not yet written: the first
    // finish into a slot overwrites it instead of accumulating.
    std::vector<char> slot_fresh;
    bool take_fresh(int slot) {
        const bool fresh = slot < int(slot_fresh.size()) && slot_fresh[slot];
        if (fresh) slot_fresh[slot] = 0;
        return fresh;
    }
    void reserve_costs(int costs);
    void reserve_grads(int layers);
    void reserve_scalars(int costs, int layers);
    // Stream capture (cpde_capture_begin .. cpde_capture_end): the calls in
    // between record their launches into a HIP graph instead of running them.
    // A recording holds raw device pointers, so it replays only while no
    // device memory of this device was released or regrown since (`layout`
    // counts those events) and while each network's active gradient buffers
    // are those it was recorded with.
    bool capturing = false;
    uint64_t layout = 0, capture_layout = 0;
    std::vector<Net*> nets;  // live networks
    struct NetCapture {
        Net* net;
        std::vector<int> active;
    };
    std::vector<NetCapture> capture_nets;  // state when the open capture began
    // Deferred gradient reductions (cpde_gradients_defer): a backward pass's
    // reduction waits so that the next pass over the same network, and the
    // scalar graph, ride in the same launch.  `partial_end` floats of the
    // network's partial buffer belong to the waiting reduction.
    bool defer = false;
    struct PendingReduce {
        bool open = false;
        Net* net = nullptr;
        ReduceArgs ra{};
        size_t partial_end = 0;
        // the weight-gradient launch waits too, before the reduction; it reads
        // the stacks its passes wrote (`plan`'s, in the network's arena, for
        // the first)
        bool wgrad = false;
        WgradArgs wa{};
        double flops = 0;
        const Plan* plan = nullptr;
    } waiting;
    // While deferring, a one-pass expression epoch is held back and launched
    // together with the next one of another plan over the same network, or
    // alone before anything else is launched that depends on it.
    std::shared_ptr<HeldEpoch> held;
};

// Synchronise the device's stream; refused while a capture is open (the
// caller allocates, frees or reads back, which a recording cannot hold).
void sync_stream(Device& d, int site = 0);
// Launch the reduction that cpde_gradients_defer keeps waiting, if any (its
// weight-gradient launch first).
void flush_reduce(Device& d);
// Launch only the waiting weight-gradient launch (the reduction may wait on).
void flush_wgrad(Device& d);

// Blocks reduce_grouped_kernel uses for a transition of `count` entries.
inline int reduce_blocks(int count, bool split_minor) { return split_minor ? (count + 3) / 4 : (count + 63) / 64; }

// Schema-specialised layer-fused kernels of one plan (jit.cpp, fused.hip.in).
struct FusedModule {
    hipModule_t module = nullptr;
    hipFunction_t input_layer = nullptr, output_backward = nullptr;
    std::vector<hipFunction_t> hidden_forward, hidden_backward;  // per transition (index t)
    hipFunction_t network_forward = nullptr, network_backward = nullptr, network_epoch = nullptr;
    int points_per_block = 2, net_points_per_block = 1, net_threads = 256;
    bool scaled = false;  // sigmoid stacks of the network kernels hold row alpha / alpha! (dE/dz: times alpha!)
    bool inkernel_wgrad = false;  // the network backward writes every hidden transition's per-block partial
    ~FusedModule();
};
std::string compose_source(const Tables& t, const std::vector<int>& splits, bool scaled = false);
// Launch-shape choices of the fused kernels (environment overrides in api.hip).
struct FusedTuning {
    int points_per_block = 2;      // layer-fused kernels
    int net_points_per_block = 1;  // network-fused kernels
    int net_threads = 256;         // network-fused kernels: lanes per workgroup (4 or 8 waves)
    int max_split = 4;             // lanes per composition, at most
    int max_split_adjoint = 1;     // lanes per adjoint composition, at most
    int alias = 0;                 // network kernels: products write over their operand tile (one LDS tile)
    int forward_blocks = 2, backward_blocks = 2;  // blocks per CU the register budget must allow
    int col_tile = 0;              // column tile of the network products: 16, 32, or 0 (chosen per shape)
    int scaled = 1;                // network kernels keep Taylor-scaled sigmoid stacks (row alpha / alpha!)
    int inkernel_wgrad = 0;        // network backward kernels write hidden weight-gradient partials themselves
    int b_pairs = 1;               // 16-column products: each wave takes 32-neuron blocks, B loaded as float2
    int tier_prio = 0, tier_cus = 256;  // one-pass epochs: wave priorities by dispatch round, and the CU count
    int stamps = 0;                // one-pass epochs write per-phase clock stamps over their output stack
};
// Whether the schema is closed under swapping variables 0 and 1 (the scaled
// forward composition then splits over two lanes, one per mirror image).
bool mirror_symmetric(const Tables& t);
std::string fused_source(const Tables& t, const std::vector<int>& neurons, const FusedTuning& tuning);
std::string expression_epoch_source(const Tables& t, const std::vector<int>& neurons, const FusedTuning& tuning,
                                    const std::string& program);
std::string expression_pair_source(const Tables& t0, const FusedTuning& u0, const std::string& program0,
                                   const Tables& t1, const FusedTuning& u1, const std::string& program1,
                                   const std::vector<int>& neurons);
// The one-pass epoch kernel of one expression program on one network module.
struct ExpressionEpoch {
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
    ~ExpressionEpoch();
};
std::vector<char> compile_module(const std::string& source, const std::string& arch, std::string* log);

// Brackets one launch with events when tracing is on.
struct TraceScope {
    Device& d;
    int index = -1;
    TraceScope(Device& dev, int kind, double work);
    ~TraceScope();
};

// ---- kernel launchers (kernels.hip) -------------------------------------------------
void launch_activate(Device& d, float* x, const float* data, int data_width, int channels, const int* rows_dev,
                     int rows, int width, int offset, int valid);
void launch_output(Device& d, float* dest, const float* out, int dest_width, int channels, const int* rows_dev,
                   int rows, int width, int offset, int valid);
void launch_compose_forward(Device& d, const Plan& p, const float* z, float* y, int n);
void launch_compose_adjoint(Device& d, const Plan& p, const float* z, float* g, int n);
// C[M x N] = A[M x K] * B[K x N]; a_t: A stored k-contiguous (A[k + lda*m]);
// b_t: B stored n-contiguous (B[n + ldb*k]).  bias (may be null) is added to every
// column n with n % period == 0.
void launch_gemm(Device& d, int M, int N, int K, const float* A, int lda, bool a_t, const float* B, int ldb, bool b_t,
                 float* C, int ldc, const float* bias, int period);
void launch_matching(Device& d, const Plan& p, const float* y, float* g, const float* target, int target_width,
                     const int* target_rows, const float* weights, int weight_samples, int offset, int valid,
                     int cost_index, bool collect, bool gradient);
void launch_polynomial(Device& d, const Plan& p, const float* y, float* g, const cpde_poly_term* terms, int term_count,
                       const float* coefficients, const float* rhs, const float* weights, int equations, int samples,
                       int offset, int valid, int cost_index, bool collect, bool gradient);
void launch_sample_reduce(Device& d, const double* values, const int* bad, int valid, int offset, int cost_index);
void launch_scale_adjoint(Device& d, const Plan& p, float* g, const double* multiplier);
void launch_costs_begin(Device& d, int costs);
// Statistics of `transitions` (<= kMaxTransitions) gradients into slots first_slot...
void launch_grad_stats(Device& d, const float* const* g, const int* counts, int transitions, int first_slot);
void launch_fill_grouped(Device& d, float* const* p, const int* counts, int buffers, float value);
// WT[t][i + n_in*o] = W[t][o + n_out*i] for `count` blocks in one launch.
void launch_transpose(Device& d, const float* const* W, float* const* WT, const int* n_in, const int* n_out,
                      int count);
// Fixed-order sum of `blocks` per-workgroup cost records into cost slot cost_index.
void launch_finish_cost(Device& d, const CostStats* partials, int blocks, int cost_index);
// Zero the slots among [0, count) still marked fresh (before something reads them on the device).
void launch_clear_fresh(Device& d, int count);
void launch_fill(Device& d, float* p, size_t count, float value);
void launch_output_forward(Device& d, const float* W, const float* Y, float* Z, int NI, int NO, int R, int columns);
void launch_wgrad_grouped(Device& d, const WgradArgs& a, double flops);
void launch_reduce_grouped(Device& d, const ReduceArgs& a);
void launch_reduce_rprop(Device& d, const ReduceArgs& a, Net& net, int first);
// RPROP over every transition, then the switch of the active gradient
// buffers; with `guard`, the update applies only where the rule accepts the
// epoch, and the switch is left to the caller.
// A copy of the scalar block to its host mirror made by an update launch.
struct ScalarPublish {
    const void* src;
    void* dst;
    size_t bytes;  // a multiple of 4
};
// test: the launch tests the gradients for finiteness itself and writes the
// gradient totals in their short form (only where update_tests(net) holds).
void launch_rprop(Device& d, Net& net, const UpdateGuard* guard = nullptr, const ScalarPublish* publish = nullptr,
                  bool test = false);
// Adam step `step`; with `guard`, only where the rule accepts the epoch.
void launch_adam(Device& d, Net& net, int step, float lr, const UpdateGuard* guard = nullptr,
                 const ScalarPublish* publish = nullptr, bool test = false);
// Whether an update launch can test the network's gradients itself: one
// transition group whose entries fit the launch's chunk table (10,240 and
// fewer, about).
bool update_tests(const Net& net);
void launch_set_steps(Device& d, Net& net, float value);
void launch_restore_steps(Device& d, Net& net, float floor_value);
GraphLaunch graph_launch(Device& d, const cpde_scalar_node* nodes, int count, int root, int leaves, double* values,
                         double* adjoints, double* multipliers, int* active, cpde_graph_summary* summary,
                         bool gradient);
void launch_graph(Device& d, const GraphLaunch& g);

}  // namespace cpde
