/*
 * cpde_hip.h -- C ABI of the MI355X (gfx950) cPDE device library, libcpde_hip.so.
 *
 * The reference drives its kernels through an in-source operator seam: the
 * CPDE_LAUNCH macro plus the cuBLAS/CUB/runtime subset that cpu/include/
 * substitutes (cuda/backend_launch.hpp:1-10, cpu/include/cublas_v2.h:23-83,
 * cpu/include/cub/device/device_reduce.cuh:1-16).  This header sits at that seam:
 * the host server (cpde_amd/csrc/server.cpp) calls only these entry points, the
 * way the reference's Server calls its network/Workspace methods.  Plain
 * pointers and sizes only; every pointer documented "device" is device memory
 * obtained from cpde_buffer_alloc (or a network/plan accessor).
 *
 * Error convention (the reference's: cuda/cuda_check_v1.cuh:36-47 exits on a
 * device fault; validation errors become kind-1 frames, cuda/cpde_server.cu:22):
 *   CPDE_OK         success
 *   CPDE_EINVAL     invalid argument -- the host reports it and keeps all state
 *   CPDE_EDEVICE    HIP runtime or kernel failure -- the host prints and exits
 *   CPDE_ECOMPILE   hipRTC rejected a generated expression kernel
 * cpde_last_error() returns the message of the calling thread's last failure.
 *
 * Layouts.  A stack holds, for one layer, every derivative row of every point of
 * a chunk: [point][row][neuron], neuron fastest.  Wire data (protocol op 2) is
 * [row][sample][channel].  A weight block is n_out x (n_in+1), column-major,
 * bias in the last column (cuda/cpde_engine.cuh:622-639).
 */
#ifndef CPDE_HIP_H
#define CPDE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CPDE_OK 0
#define CPDE_EINVAL 1
#define CPDE_EDEVICE 2
#define CPDE_ECOMPILE 4

typedef struct cpde_device_s cpde_device;
typedef struct cpde_net_s cpde_net;
typedef struct cpde_plan_s cpde_plan;
typedef struct cpde_program_s cpde_program;
typedef struct cpde_stacks_s cpde_stacks;
typedef struct cpde_replay_s cpde_replay;

/* Per-cost reduction result: signed double sum and the first bad (sample,
 * component); component -1 means the objective itself
 * (cuda/reduction_kernels.cuh:28-46).  INT32_MAX marks "no bad value". */
typedef struct {
    double value;
    int32_t bad_sample;
    int32_t bad_component;
} cpde_cost_stats;

/* Per-layer gradient statistics (cuda/reduction_kernels.cuh:53-58,81-98). */
typedef struct {
    double squared_norm;
    double max_abs;
    uint64_t nonfinite_count;
    int32_t first_nonfinite;
    int32_t pad_;
} cpde_gradient_stats;

/* Sparse polynomial residual term (cuda/cost_kernels.cuh:37): b = -1 is linear. */
typedef struct {
    int32_t equation, a, b;
} cpde_poly_term;

/* Scalar graph node (cuda/scalar_ops.cuh:6). */
typedef struct {
    int32_t op, a, b, pad_;
    double parameter;
} cpde_scalar_node;

/* Scalar graph result (cuda/cost_graph.cuh:6). */
typedef struct {
    double value;
    int32_t bad_node;
    int32_t pad_;
} cpde_graph_summary;

const char* cpde_last_error(void);

/* ---- device, stream and buffers (replaces cudaSetDevice/cudaStreamCreate/
 *      cudaMalloc/cudaMemcpy uses, cuda/cpde_engine.cuh:23-87, cuda/cpde_server.cu:26-33) */
int cpde_device_open(int ordinal, cpde_device** out);
int cpde_device_close(cpde_device* dev);
int cpde_device_synchronize(cpde_device* dev);
/* Name and compute-unit count of the open device. */
int cpde_device_info(cpde_device* dev, char* name, size_t capacity, int* compute_units);
int cpde_buffer_alloc(cpde_device* dev, size_t bytes, void** out);
int cpde_buffer_free(cpde_device* dev, void* ptr);
/* Synchronous copies in stream order. */
int cpde_buffer_upload(cpde_device* dev, void* dst, const void* src, size_t bytes);
int cpde_buffer_download(cpde_device* dev, void* dst, const void* src, size_t bytes);
int cpde_buffer_copy(cpde_device* dev, void* dst, const void* src, size_t bytes);

/* ---- network: weights and optimizer state (class weights/network,
 *      cuda/cpde_engine.cuh:562-659,782-850; op 3 cuda/cpde_server.cu:455-473).
 * initial[t] is the n_{t+1} x (n_t+1) block of transition t (may be NULL: zeros).
 * Gradient buffers start at zero and the RPROP step at 0.002. */
int cpde_net_create(cpde_device* dev, int layers, const int* neurons, const int* linear,
                    const float* const* initial, cpde_net** out);
int cpde_net_destroy(cpde_net* net);
/* Device pointer and element count of state buffer b of transition t:
 * 0 weights, 1 and 2 the gradient ping-pong pair, 3 RPROP step / Adam first moment.
 * Weights written through a buffer-0 pointer are seen by the next library call
 * on the network: write them before that call, or ask for the pointer again
 * after writing (the library keeps a transposed copy of the weights, which it
 * rebuilds after the pointer has been handed out). */
int cpde_net_state(cpde_net* net, int transition, int buffer, float** device_ptr, int* count);
/* The active gradient buffer (1 or 2) of a transition (weights::act_grad). */
int cpde_net_active(cpde_net* net, int transition);
int cpde_net_set_active(cpde_net* net, int transition, int active);
/* Incremented whenever the network's stack arena is reallocated (all plans'
 * stacks are then undefined until the next cpde_activate). */
uint64_t cpde_net_generation(cpde_net* net);

/* ---- plans: one derivative schema x chunk width x backward flag over a network
 *      (class context + stack + derivative_tables, cuda/cpde_engine.cuh:391-560;
 *      Server::prepare, cuda/cpde_server.cu:148-157).
 * table: rows x (variables+1), row-major (order, counts...); orders sorted,
 * value row first, order <= 6. */
int cpde_plan_create(cpde_net* net, int rows, int variables, const int* table, int width, int backward,
                     cpde_plan** out);
int cpde_plan_destroy(cpde_plan* plan);
/* Device pointer of a plan's stack: kind 0 = z (layer 0: the input), 1 = y
 * (sigmoid activations), 2 = adjoint dE/dz, 3 = u, the jet of sigma'(z) (the
 * reference's DPlus rows, cuda/derivative_kernels_v4.cu:12-380, with u[0] =
 * sigma'(z0)).  Network-fused plans keep u instead of z for sigmoid layers
 * (their adjoint needs only u); other plans keep z.  Layout [point][row][neuron]. */
int cpde_plan_stack(cpde_plan* plan, int layer, int kind, float** device_ptr);
/* Network-fused plans keep sigmoid layers' stacks Taylor-scaled: row alpha of y
 * and u holds d^alpha / alpha!, and of dE/dz holds alpha! dE/dz_alpha (the
 * adjoint of the scaled rows).  This fills row_factor[rows] with the factor
 * that turns a stored row into the reference's row (all ones for unscaled
 * stacks).  No counterpart in the reference, whose stacks are unscaled; for
 * callers that inspect stacks. */
int cpde_plan_stack_scale(cpde_plan* plan, int layer, int kind, float* row_factor);
/* Retained forward results.  A stack set is a plan's own copy of every layer's
 * stacks and of its activated input chunk; cpde_plan_bind(plan, set) makes the
 * plan's launches (activate, forward, costs, backward) use the set in place of
 * the network's shared arena until cpde_plan_bind(plan, NULL) or another bind.
 * A forward into a bound set stays there while other chunks and plans run, so a
 * later backward needs no second forward: the retention the reference plans
 * for costs with value-dependent multipliers (IMPLEMENTATION_PLAN.md:750-831,
 * not implemented in its engine, which recomputes those forwards and keeps
 * only the last chunk's, cuda/cpde_server.cu:273-318).  While a set is bound,
 * other plans of the network must not run.  Destroying a bound set, its plan or
 * its network unbinds it first. */
int cpde_stacks_create(cpde_plan* plan, cpde_stacks** out);
int cpde_plan_bind(cpde_plan* plan, cpde_stacks* stacks);
int cpde_stacks_destroy(cpde_stacks* stacks);

/* ---- hot path ---------------------------------------------------------------------- */
/* Server::activate (cuda/cpde_server.cu:158-170): copy the chunk's rows of wire
 * data [data_rows][data_width][channels] (device) into layer 0, rows[r] (host)
 * selecting the data row of plan row r; lanes [valid, width) are zeroed. */
int cpde_activate(cpde_plan* plan, const float* data, int data_width, const int* rows, int offset, int valid);
/* network::feedforward (cuda/cpde_engine.cuh:889-913): every layer's linear step
 * (fp32 MFMA, bias on the value row) and sigmoid composition through order 6. */
int cpde_forward(cpde_plan* plan);
/* Copy the output stack's valid lanes to wire layout dest [dest_rows][dest_width][n_out]
 * (device), plan row r going to dest row rows[r] (Server::evaluate :171-183). */
int cpde_output(cpde_plan* plan, float* dest, int dest_width, const int* rows, int offset, int valid);

/* Reset cost slots [0, costs) (Workspace::begin, cuda/reduction_kernels.cuh:149-152). */
int cpde_costs_begin(cpde_device* dev, int costs);
/* Deferred gradient reductions.  No counterpart in the reference, whose
 * backward passes each end in their own accumulating GEMMs.  While on, the
 * reduction that ends a backward pass (cpde_backward, cpde_epoch_matching,
 * cpde_epoch_expression) waits: the next backward pass over the same network
 * that accumulates onto it joins it, and the two are reduced in one launch,
 * bit for bit as two launches in turn; cpde_graph_execute then rides in that
 * launch after its cost finishes.  A one-pass expression epoch is held back
 * too, and the next one of another plan over the same network shares its
 * launch.  Every call that reads gradients, costs or the device (downloads,
 * statistics, optimizers, synchronisation, another cost into a slot the
 * waiting launch finishes) launches them first, and so does turning deferral
 * off. */
int cpde_gradients_defer(cpde_device* dev, int on);
/* Array-matching squared loss (cuda/cost_kernels.cuh:6-35) fused with its
 * deterministic reduction into cost slot cost_index.  target: device wire data
 * [target_rows_total][target_width][n_out]; target_rows, weights: device. */
int cpde_cost_matching(cpde_plan* plan, const float* target, int target_width, const int* target_rows,
                       const float* weights, int weight_samples, int offset, int valid, int cost_index,
                       int collect, int gradient);
/* One chunk of Server::pass for an array-matching cost with gradient
 * (cuda/cpde_server.cu:223-257): cpde_forward, cpde_cost_matching(gradient=1)
 * and cpde_backward(accumulate) with the same arguments.  The reference runs
 * them as separate launches; on the network-fused kernels, when the chunk's
 * workgroups fit on the device together, this is one launch (a point's
 * matching terms depend on that point alone), the cost's finish and the
 * weight-gradient contraction.  The input chunk must be activated.  That one
 * launch leaves two stacks unwritten, which no later launch reads: y of the
 * last hidden layer and dE/dz of the first (cpde_plan_stack kinds 1 and 2);
 * read them after the separate calls instead. */
int cpde_epoch_matching(cpde_plan* plan, const float* target, int target_width, const int* target_rows,
                        const float* weights, int weight_samples, int offset, int valid, int cost_index, int collect,
                        int accumulate);
/* cpde_epoch_matching followed by cpde_rprop, with the split reduction of the
 * weight gradients and the RPROP update in one launch (one launch fewer per
 * epoch); the gradients, weights and optimizer state end bit-identical to the
 * two calls.  No counterpart in the reference, whose training step launches
 * them separately (cuda/cpde_server.cu:384-409); for callers that update after
 * every epoch of a single matching cost (the last chunk of the epoch). */
int cpde_epoch_matching_rprop(cpde_plan* plan, const float* target, int target_width, const int* target_rows,
                              const float* weights, int weight_samples, int offset, int valid, int cost_index,
                              int collect, int accumulate);
/* cpde_epoch_matching that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The same kernels as cpde_epoch_matching's one-pass epoch, with the same
 * results; the per-workgroup cost records and the weight-gradient split
 * partials live in the library's static device scratch of
 * CPDE_STATIC_SCRATCH_BYTES, which every GPU the library runs on holds until
 * the process ends, instead of buffers grown on demand.  Refused with
 * CPDE_EINVAL, before any launch: a plan whose one-pass epoch does not apply
 * (network-fused kernels, the chunk's workgroups resident together), a plan
 * needing more scratch than that, a cost slot not reserved by
 * cpde_costs_begin, or kernel tracing on.  Every call on one GPU shares its
 * scratch: calls that overlap on one GPU (from different device handles or
 * threads) race. */
#define CPDE_STATIC_SCRATCH_BYTES (16u << 20)
int cpde_epoch_matching_static(cpde_plan* plan, const float* target, int target_width, const int* target_rows,
                               const float* weights, int weight_samples, int offset, int valid, int cost_index,
                               int collect, int accumulate);
/* Sparse linear/quadratic residual cost (cuda/cost_kernels.cuh:37-90); all device. */
int cpde_cost_polynomial(cpde_plan* plan, const cpde_poly_term* terms, int term_count, const float* coefficients,
                         const float* rhs, const float* weights, int equations, int samples, int offset, int valid,
                         int cost_index, int collect, int gradient);
/* dE/dY *= multiplier for graph leaves (cuda/cost_graph.cuh:29-34); device scalar. */
int cpde_scale_adjoint(cpde_plan* plan, const double* multiplier);
/* network::backprop (cuda/cpde_engine.cuh:947-991): adjoint compositions, the
 * transposed products and the weight+bias gradient contraction (deterministic
 * split-K).  accumulate=0 overwrites the active gradient, 1 adds to it. */
int cpde_backward(cpde_plan* plan, int accumulate);

/* ---- reductions, validation data and optimizer ------------------------------------- */
/* Per-transition statistics of the active gradient into slot t (inspect_gradients). */
int cpde_inspect_gradients(cpde_net* net);
/* Synchronous download of cost slots and gradient-statistics slots (Workspace::download). */
int cpde_scalars_download(cpde_device* dev, int costs, cpde_cost_stats* cost_out, int layers,
                          cpde_gradient_stats* gradient_out);
/* The same, plus a scalar graph's summary (device, written by cpde_graph_execute)
 * in the same synchronisation: one host round trip per graph epoch, as the
 * reference queues the graph copy before its scalar download
 * (cuda/cpde_server.cu:317, cuda/reduction_kernels.cuh:171-177).  summary NULL
 * (summary_out not NULL): the device's own summary slot, downloaded in the same
 * copy as the cost and gradient slots. */
int cpde_scalars_download_graph(cpde_device* dev, int costs, cpde_cost_stats* cost_out, int layers,
                                cpde_gradient_stats* gradient_out, const cpde_graph_summary* summary,
                                cpde_graph_summary* summary_out);
/* RPROP over every transition, then switch the active gradient buffer
 * (Resile_k + switch_active, cuda/derivative_kernels_v4.cu:752-778). */
int cpde_rprop(cpde_net* net);
/* The training epoch's scalar download and its RPROP update in one call
 * (cuda/cpde_server.cu:394-410, the download, the checks and Resile_k):
 * cpde_update_issue, then cpde_update_resolve. */
int cpde_scalars_download_rprop(cpde_device* dev, int costs, cpde_cost_stats* cost_out, int layers,
                                cpde_gradient_stats* gradient_out, cpde_graph_summary* summary_out, cpde_net* net,
                                int* updated);
/* The first half of that call: the update -- method 0 RPROP, 1 Adam step
 * `step` with rate lr (ADAM_k, cuda/derivative_kernels_v4.cu:780-799) --
 * which applies only if every cost is finite with no bad sample, the graph has
 * no bad node and every gradient is finite: the checks after which the server
 * updates.  Its launch also copies `costs` cost totals, the gradient totals of
 * every transition (layers = the network's transitions) and, with with_graph,
 * the device's graph summary to the device's host block, and leaves its
 * verdict on the device, where reductions launched before the resolution read
 * it and store into this network's gradient buffers only if it applied.
 * RPROP's active gradient buffers switch now, in expectation, so that calls
 * made before the resolution (the next epoch's first passes) write the next
 * gradient where it belongs.  costs <= 64; one issued update per device at a
 * time. */
int cpde_update_issue(cpde_device* dev, int costs, int layers, int with_graph, cpde_net* net, int method, int step,
                      float lr);
/* cpde_inspect_gradients(net), then cpde_update_issue, as one call (the
 * reference takes the statistics and then updates, cuda/cpde_server.cu:394-410,
 * with no call of its own for the pair).  With full_stats = 0, on a network of
 * one transition group whose weights and biases fit the launch's chunk table
 * (40 chunks of 256 per transition group, about 10,240 entries), the update
 * launch tests the gradients for finiteness itself instead, and the gradient
 * totals it hands out are short: nonfinite_count 1 where the transition has a
 * non-finite entry (else 0), first_nonfinite none, squared norm and maximum 0.
 * The verdict is the same; for whole statistics of a rejected epoch, call
 * cpde_inspect_gradients afterwards (the gradients are untouched). */
int cpde_inspect_update_issue(cpde_device* dev, int costs, int layers, int with_graph, cpde_net* net, int method,
                              int step, float lr, int full_stats);
/* The second half: wait for that launch, hand out the scalars (as
 * cpde_scalars_download_graph does) and say whether the update applied; where
 * it did not, RPROP's buffers switch back. */
int cpde_update_resolve(cpde_device* dev, cpde_cost_stats* cost_out, cpde_gradient_stats* gradient_out,
                        cpde_graph_summary* summary_out, int* updated);
/* No counterpart in the reference (it has no deferred launches).  Drop the
 * held one-pass epoch and the waiting weight-gradient and reduction launches
 * without launching them, and stop deferring (cpde_gradients_defer):
 * for passes issued ahead of a check that then rejected the epoch before them.
 * Such passes write scratch (stacks, records, partials), and the reductions
 * they had to launch stored nothing into a network whose issued update did not
 * apply, so nothing of the network's state changes. */
int cpde_gradients_discard(cpde_device* dev);
/* Adam step `step` (>= 1) with learning rate lr (ADAM_k, :780-799). */
int cpde_adam(cpde_net* net, int step, float lr);
/* Set every step to value and clear both histories (Set_Resile_k, :825-832). */
int cpde_set_steps(cpde_net* net, float value);
/* Raise steps below floor to floor, clearing that entry's histories (Reset_Resile_k). */
int cpde_restore_steps(cpde_net* net, float floor_value);
/* Zero the active gradient (graph passes, cuda/cpde_server.cu:278). */
int cpde_zero_gradient(cpde_net* net);
/* Zero gradients and steps/moments, active = 1 (Server::reset, :184-192). */
int cpde_reset_optimizer(cpde_net* net);

/* ---- scalar-expression costs: generated source compiled with hipRTC for gfx950
 *      (cuda/expression_program.hpp:96-131 used NVRTC) and the scalar cost graph.
 * The source defines the kernel `expression` (arguments as cpde_cost_expression
 * passes them) and may define the per-sample functions cpde_expression_inputs
 * (a sample's quadrature weight and field values, gathered from global memory)
 * and cpde_expression_point (value, flag and adjoint from those inputs and the
 * sample's outputs), which cpde_epoch_expression compiles into the network
 * kernels. */
int cpde_program_compile(cpde_device* dev, const char* source, cpde_program** out, char* log, size_t log_capacity);
int cpde_program_destroy(cpde_program* program);
/* Per-sample expression over the plan's output stack, then its deterministic
 * reduction into cost slot cost_index.  fields [F][samples], quadrature_weights
 * [samples] (device, double); multiplier: device double or NULL;
 * scratch: device, 2*width doubles' worth (values + flags). */
int cpde_cost_expression(cpde_plan* plan, cpde_program* program, const double* fields,
                         const double* quadrature_weights, int samples, int offset, int valid,
                         const double* multiplier, void* scratch, int cost_index, int collect, int gradient);
/* One chunk of Server::pass for an expression cost with gradient
 * (cuda/cpde_server.cu:223-257): cpde_forward, cpde_cost_expression(gradient=1)
 * and cpde_backward(accumulate) with the same arguments.  On the network-fused
 * kernels, when the chunk's workgroups fit on the device together and the
 * program defines both per-sample functions, this is one launch (a sample's value
 * and adjoint depend on that sample alone; the program is compiled into the
 * network module on first use), the cost's finish and the weight-gradient
 * contraction.  The multiplier must be final when the call is made.  The input
 * chunk must be activated.  The one launch leaves the same two stacks
 * unwritten as cpde_epoch_matching's. */
int cpde_epoch_expression(cpde_plan* plan, cpde_program* program, const double* fields,
                          const double* quadrature_weights, int samples, int offset, int valid,
                          const double* multiplier, void* scratch, int cost_index, int collect, int accumulate);
/* Whether cpde_epoch_expression runs (plan, program) as one launch (1) or as
 * its three separate steps (0).  No counterpart in the reference: the server
 * asks it when it chooses between keeping a chunk's forward for a later
 * backward and recomputing it inside that launch. */
int cpde_epoch_expression_fused(cpde_plan* plan, cpde_program* program, int* fused);
/* cost_graph::execute (cuda/cost_graph.cuh:6-27) on one lane: reads cost slots,
 * writes values/adjoints/multipliers/active (device) and the summary (device;
 * NULL: the device's own summary slot, see cpde_scalars_download_graph). */
int cpde_graph_execute(cpde_device* dev, const cpde_scalar_node* nodes, int count, int root, int leaves,
                       double* values, double* adjoints, double* multipliers, int* active,
                       cpde_graph_summary* summary, int gradient);

/* Compile the schema-specialised fused kernels of (schema, architecture) for
 * chunks of `width` points (0: any) on a device of `compute_units` CUs, for a
 * GPU architecture (e.g. "gfx950"), into the on-disk code-object cache,
 * without a device.  The reference's analogue is its per-expression NVRTC
 * compile (cuda/expression_program.hpp:104-121), done lazily at first use. */
int cpde_jit_prepare(int rows, int variables, const int* table, int layers, const int* neurons, int width,
                     int compute_units, const char* arch, char* log, size_t log_capacity);

/* ---- captured epochs ------------------------------------------------------------- */
/* No counterpart in the reference, whose server issues every launch of every
 * epoch from the host.  Between cpde_capture_begin and cpde_capture_end the
 * calls on `dev` record their launches into a HIP graph instead of running
 * them; their host-side bookkeeping still happens.  Calls that would
 * synchronise the device (allocation, release, read-back) are refused with
 * CPDE_EINVAL while a capture is open, and so are tracing and marks: run a
 * sequence once uncaptured so that its buffers exist before recording it.
 * cpde_capture_end(keep = 1) instantiates the recording and runs it once, so
 * the recorded calls complete as if they had run; keep = 0, or any failure,
 * discards it and undoes the bookkeeping that depends on the device work (the
 * active gradient buffers).  cpde_replay_launch runs the recording again on
 * the device stream.  It is refused, without launching, once device memory
 * of the device has been released or regrown since the capture, or when a
 * network's active gradient buffers are not those it was recorded with (an
 * optimizer update flips them: record one replay per parity).  Kernel
 * arguments are fixed at capture: what a replay reads and writes are the
 * buffers the recorded calls named, with their contents at replay time. */
int cpde_capture_begin(cpde_device* dev);
int cpde_capture_end(cpde_device* dev, int keep, cpde_replay** out);
int cpde_replay_launch(cpde_replay* replay);
int cpde_replay_destroy(cpde_replay* replay);

/* ---- timing ---------------------------------------------------------------------- */
/* Kernel tracing (no counterpart in the reference, which has no built-in
 * profiling): while enabled, every launch is bracketed by HIP events on the
 * device stream and accounted to its kernel class.  Enabling (or disabling)
 * clears the totals.  cpde_trace_read synchronizes and returns a class's
 * launch count, summed device milliseconds and summed algorithmic work
 * (bytes for HBM-bound classes, flops for the matrix-core classes). */
int cpde_trace_enable(cpde_device* dev, int on);
int cpde_trace_read(cpde_device* dev, int kind, uint64_t* launches, double* total_ms, double* work);
const char* cpde_trace_name(int kind);
int cpde_trace_kinds(void);
/* Record an event on the device stream; elapsed milliseconds between two marks. */
int cpde_mark(cpde_device* dev, int slot);
int cpde_elapsed(cpde_device* dev, int from_slot, int to_slot, float* ms);

#ifdef __cplusplus
}
#endif
#endif
