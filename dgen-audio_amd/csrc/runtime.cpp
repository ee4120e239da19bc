// libdgen_hip runtime: context, arena + pinned host mirror, schedule,
// streams, timing.  The C ABI is declared in include/dgen_hip.h.
//
// Design notes
// - One device arena per context (hipMalloc once at configure), addressed
//   by float offsets: the reference's flat `memory` of cells
//   (Sources/DGen/Compilation/MemoryAllocation.swift:4-24).  The reference
//   relies on host-coherent storage (MetalRuntime.swift:232); on discrete HBM
//   the host mirror is pinned and moved only by explicit upload/download.
// - Stream 0 carries the schedule; ops flagged SIDE run on a second stream
//   (default priority) that first waits for the run's start event (or, for a
//   SIDE|FORK op, for stream 0's work enqueued before it), and a JOIN op
//   makes stream 0 wait for the side stream before it launches.
// - run() is synchronous like MetalCompiledKernel.run (commit+wait,
//   MetalRuntime.swift:334-337).
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "dgen_process_v1.h"
#include "internal.h"

namespace dgen {

static thread_local char g_err[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_cell(const Launch& L, int64_t off, uint64_t n, const char* what) {
  if (off < 0 || (uint64_t)off > L.arena_floats || n > L.arena_floats - (uint64_t)off)
    return fail(DGEN_HIP_E_RANGE, "%s: cell range [%lld, +%llu) outside arena of %llu floats", what,
                (long long)off, (unsigned long long)n, (unsigned long long)L.arena_floats);
  return 0;
}

static Launcher launcher_for(uint32_t k) {
  switch (k) {
    case DGEN_HIP_K_ACCUM_TABLE: return launch_accum_table;
    case DGEN_HIP_K_DENSE_SMALL: return launch_dense_small;
    case DGEN_HIP_K_GEMM: return launch_gemm;
    case DGEN_HIP_K_HEADS_FWD: return launch_heads_fwd;
    case DGEN_HIP_K_PHASOR_CARRY: return launch_phasor_carry;
    case DGEN_HIP_K_SYNTH_FWD: return launch_synth_fwd;
    case DGEN_HIP_K_SPECTRAL_LOSS: return launch_spectral_loss;
    case DGEN_HIP_K_SPECTRAL_GATHER: return launch_spectral_gather;
    case DGEN_HIP_K_SYNTH_BWD: return launch_synth_bwd;
    case DGEN_HIP_K_SYNTH_BWD_REDUCE: return launch_synth_bwd_reduce;
    case DGEN_HIP_K_HEADS_BWD: return launch_heads_bwd;
    case DGEN_HIP_K_COLSUM: return launch_colsum;
    case DGEN_HIP_K_DENSE_SMALL_WGRAD: return launch_dense_small_wgrad;
    case DGEN_HIP_K_ADAM: return launch_adam;
    case DGEN_HIP_K_OSC_BANK: return launch_osc_bank;
    case DGEN_HIP_K_NOISE_TABLE: return launch_noise_table;
    case DGEN_HIP_K_ROW_SCHEDULE: return launch_row_schedule;
    case DGEN_HIP_K_FFT_TABLES: return launch_fft_tables;
    case DGEN_HIP_K_LERP_FRAMES: return launch_lerp_frames;
    case DGEN_HIP_K_BIQUAD_CHUNK: return launch_biquad_chunk;
    case DGEN_HIP_K_BIQUAD_CARRY: return launch_biquad_carry;
    case DGEN_HIP_K_BIQUAD_FWD: return launch_biquad_fwd;
    case DGEN_HIP_K_BIQUAD_ADJ_CHUNK: return launch_biquad_adj_chunk;
    case DGEN_HIP_K_BIQUAD_BWD: return launch_biquad_bwd;
    case DGEN_HIP_K_STFT_FWD: return launch_stft_fwd;
    case DGEN_HIP_K_STFT_BWD: return launch_stft_bwd;
    case DGEN_HIP_K_MEMBRANE_FWD: return launch_membrane_fwd;
    case DGEN_HIP_K_MEMBRANE_BWD: return launch_membrane_bwd;
    case DGEN_HIP_K_STREAM_OSC_BANK: return launch_stream_osc_bank;
    case DGEN_HIP_K_STREAM_BIQUAD: return launch_stream_biquad;
    case DGEN_HIP_K_TEMPORAL_GRAD_SCAN: return launch_temporal_grad_scan;
    case DGEN_HIP_K_SWEPT_PHASOR: return launch_swept_phasor;
    case DGEN_HIP_K_SVF_CHUNK: return launch_svf_chunk;
    case DGEN_HIP_K_SVF_FWD: return launch_svf_fwd;
    case DGEN_HIP_K_SVF_SEQ:
    case DGEN_HIP_K_STREAM_SVF: return launch_svf_seq;
    case DGEN_HIP_K_SVF_ADJ_CHUNK: return launch_svf_adj_chunk;
    case DGEN_HIP_K_SVF_BWD: return launch_svf_bwd;
    case DGEN_HIP_K_SPLIT_BF16: return launch_split_bf16;
    case DGEN_HIP_K_UOP_BLOCK: return launch_uop_block;
    case DGEN_HIP_K_RUN_TABLE: return launch_run_table;
    default: return nullptr;
  }
}

}  // namespace dgen

using namespace dgen;

struct dgen_hip_ctx {
  int device = 0;
  int cu_count = 256;
  hipStream_t s0 = nullptr, s1 = nullptr;
  hipEvent_t ev_start = nullptr, ev_side = nullptr, ev_fork = nullptr;
  float* d_arena = nullptr;
  float* h_arena = nullptr;
  uint64_t floats = 0;
  uint32_t max_frames = 0;
  std::vector<dgen_hip_op> ops;
  bool configured = false;
  // graph replay of the per-run schedule (dgen_hip_set_graphs)
  bool use_graphs = false;
  hipGraphExec_t graph = nullptr;
  uint32_t graph_frames = 0;
  // host sample rate of the runs (dgen_hip_set_sample_rate; 0: each op's own)
  float host_sr = 0.f;
  // output cells (dgen_hip_set_outputs), downloaded by every dgen_hip_run
  uint64_t out_off = 0, out_n = 0;
  // process ports (dgen_hip_set_process_ports): channel c, frame i at cell
  // in_cell[c] + i * in_stride[c] (inputs) / out_cell[c] + i * out_stride[c]
  std::vector<uint64_t> in_cell, out_cell;
  std::vector<uint32_t> in_stride, out_stride;
  // the next enqueue starts the streaming classes from zero state
  bool reset_next = false;
  // a dgen_hip_run_async whose declared outputs the next dgen_hip_sync downloads
  bool outputs_pending = false;
  // generic UOp blocks (dgen_hip_set_blocks): their loaded module and kernels
  hipModule_t blk_module = nullptr;
  std::vector<BlockInfo> blocks;
};

static int set_device(dgen_hip_ctx* c) {
  DGEN_HIP_TRY(hipSetDevice(c->device));
  return 0;
}

static Launch make_launch(dgen_hip_ctx* c, hipStream_t s, uint32_t frames, bool dry) {
  Launch L;
  L.stream = s;
  L.arena = c->d_arena;
  L.arena_floats = c->floats;
  L.frames = frames;
  L.device = c->device;
  L.cu_count = c->cu_count;
  L.blocks = c->blocks.empty() ? nullptr : c->blocks.data();
  L.n_blocks = c->blocks.size();
  L.dry = dry;
  L.host_sr = c->host_sr;
  L.reset = c->reset_next;
  return L;
}

static void drop_graph(dgen_hip_ctx* c) {
  if (c->graph) (void)hipGraphExecDestroy(c->graph);
  c->graph = nullptr;
  c->graph_frames = 0;
}

static void release_arena(dgen_hip_ctx* c) {
  drop_graph(c);
  if (c->d_arena) (void)hipFree(c->d_arena);
  if (c->h_arena) (void)hipHostFree(c->h_arena);
  c->d_arena = nullptr;
  c->h_arena = nullptr;
  c->floats = 0;
  c->out_off = c->out_n = 0;
  c->in_cell.clear();
  c->out_cell.clear();
  c->in_stride.clear();
  c->out_stride.clear();
  c->configured = false;
}

// Enqueue ops [0, n) that match `static_pass`; optional per-op event timing.
static int enqueue(dgen_hip_ctx* c, uint32_t frames, bool static_pass, std::vector<hipEvent_t>* evs) {
  DGEN_HIP_TRY(hipEventRecord(c->ev_start, c->s0));
  DGEN_HIP_TRY(hipStreamWaitEvent(c->s1, c->ev_start, 0));
  bool side_used = false;
  for (size_t i = 0; i < c->ops.size(); ++i) {
    const dgen_hip_op& op = c->ops[i];
    bool is_static = (op.flags & DGEN_HIP_OP_STATIC) != 0;
    if (is_static != static_pass) continue;
    if (op.flags & DGEN_HIP_OP_JOIN) {
      DGEN_HIP_TRY(hipEventRecord(c->ev_side, c->s1));
      DGEN_HIP_TRY(hipStreamWaitEvent(c->s0, c->ev_side, 0));
    }
    if ((op.flags & DGEN_HIP_OP_FORK) && (op.flags & DGEN_HIP_OP_SIDE)) {
      // each wait is enqueued right after its record, so one event serves
      // every fork point of the run (graph capture turns each pair into an
      // edge from stream 0's last node)
      DGEN_HIP_TRY(hipEventRecord(c->ev_fork, c->s0));
      DGEN_HIP_TRY(hipStreamWaitEvent(c->s1, c->ev_fork, 0));
    }
    hipStream_t s = (op.flags & DGEN_HIP_OP_SIDE) ? c->s1 : c->s0;
    side_used |= (s == c->s1);
    Launch L = make_launch(c, s, frames, false);
    if (evs) DGEN_HIP_TRY(hipEventRecord((*evs)[2 * i], s));
    int rc = launcher_for(op.kernel)(L, op);
    if (rc) return rc;
    if (evs) DGEN_HIP_TRY(hipEventRecord((*evs)[2 * i + 1], s));
  }
  // Never leave side-stream work unjoined past the end of a run.
  if (side_used) {
    DGEN_HIP_TRY(hipEventRecord(c->ev_side, c->s1));
    DGEN_HIP_TRY(hipStreamWaitEvent(c->s0, c->ev_side, 0));
  }
  return 0;
}

// One run of the per-run schedule.  With graphs on, the schedule for this
// frame count is captured once from both streams (the side stream joins the
// capture through the fork event and is joined back before it ends) and
// replayed with one launch; captures hold kernel launches and events only.
static int launch_run(dgen_hip_ctx* c, uint32_t frames) {
  if (!c->use_graphs) return enqueue(c, frames, false, nullptr);
  if (!c->graph || c->graph_frames != frames) {
    drop_graph(c);
    DGEN_HIP_TRY(hipStreamBeginCapture(c->s0, hipStreamCaptureModeThreadLocal));
    int rc = enqueue(c, frames, false, nullptr);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(c->s0, &g);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return fail(DGEN_HIP_E_DEVICE, "run: graph capture failed: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(&c->graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
      c->graph = nullptr;
      return fail(DGEN_HIP_E_DEVICE, "run: graph instantiation failed: %s", hipGetErrorString(e));
    }
    c->graph_frames = frames;
  }
  DGEN_HIP_TRY(hipGraphLaunch(c->graph, c->s0));
  return 0;
}

static int run_static(dgen_hip_ctx* c);

extern "C" {

int dgen_hip_abi_version(void) { return DGEN_HIP_ABI_VERSION; }

int dgen_hip_device_count(int* out) {
  if (!out) return fail(DGEN_HIP_E_INVALID, "device_count: null out");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *out = 0;
    return fail(DGEN_HIP_E_DEVICE, "hipGetDeviceCount: %s", hipGetErrorString(e));
  }
  *out = n;
  return 0;
}

const char* dgen_hip_last_error(void) { return g_err; }

int dgen_hip_create(int device, dgen_hip_ctx** out) {
  if (!out) return fail(DGEN_HIP_E_INVALID, "create: null out");
  *out = nullptr;
  int n = 0;
  DGEN_HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(DGEN_HIP_E_INVALID, "create: device %d of %d", device, n);
  dgen_hip_ctx* c = new (std::nothrow) dgen_hip_ctx();
  if (!c) return fail(DGEN_HIP_E_NOMEM, "create: out of host memory");
  c->device = device;
  int rc = set_device(c);
  if (!rc) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) c->cu_count = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&c->s0, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&c->s1, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_start, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_side, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming) != hipSuccess)
      rc = fail(DGEN_HIP_E_DEVICE, "create: stream/event creation failed");
  }
  if (rc) {
    dgen_hip_destroy(c);
    return rc;
  }
  *out = c;
  return 0;
}

static void process_unbind_if(dgen_hip_ctx* c);

int dgen_hip_destroy(dgen_hip_ctx* c) {
  if (!c) return 0;
  process_unbind_if(c);
  (void)hipSetDevice(c->device);
  if (c->s0) (void)hipStreamSynchronize(c->s0);
  if (c->s1) (void)hipStreamSynchronize(c->s1);
  release_arena(c);
  if (c->blk_module) (void)hipModuleUnload(c->blk_module);
  if (c->ev_start) (void)hipEventDestroy(c->ev_start);
  if (c->ev_side) (void)hipEventDestroy(c->ev_side);
  if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
  if (c->s0) (void)hipStreamDestroy(c->s0);
  if (c->s1) (void)hipStreamDestroy(c->s1);
  delete c;
  return 0;
}

int dgen_hip_configure(dgen_hip_ctx* c, const dgen_hip_op* ops, uint32_t n_ops, uint64_t memory_floats,
                       uint32_t max_frames) {
  if (!c) return fail(DGEN_HIP_E_INVALID, "configure: null context");
  if (n_ops && !ops) return fail(DGEN_HIP_E_INVALID, "configure: null ops");
  if (memory_floats == 0) return fail(DGEN_HIP_E_INVALID, "configure: empty arena");
  int rc = set_device(c);
  if (rc) return rc;
  DGEN_HIP_TRY(hipStreamSynchronize(c->s0));
  DGEN_HIP_TRY(hipStreamSynchronize(c->s1));
  release_arena(c);
  // Validate the schedule before allocating (dry launches need sizes only).
  c->floats = memory_floats;
  for (uint32_t i = 0; i < n_ops; ++i) {
    Launcher f = launcher_for(ops[i].kernel);
    if (!f) return fail(DGEN_HIP_E_INVALID, "configure: op %u has unknown kernel class %u", i, ops[i].kernel);
    Launch L = make_launch(c, c->s0, max_frames, true);
    rc = f(L, ops[i]);
    if (rc) {
      std::string msg = g_err;
      c->floats = 0;
      return fail(rc, "configure: op %u (kernel %u): %s", i, ops[i].kernel, msg.c_str());
    }
  }
  c->floats = 0;
  size_t bytes = (size_t)memory_floats * sizeof(float);
  if (hipMalloc(&c->d_arena, bytes) != hipSuccess) {
    c->d_arena = nullptr;
    return fail(DGEN_HIP_E_NOMEM, "configure: hipMalloc of %zu bytes failed", bytes);
  }
  if (hipHostMalloc(&c->h_arena, bytes, hipHostMallocDefault) != hipSuccess) {
    c->h_arena = nullptr;
    release_arena(c);
    return fail(DGEN_HIP_E_NOMEM, "configure: pinned host allocation of %zu bytes failed", bytes);
  }
  c->floats = memory_floats;
  memset(c->h_arena, 0, bytes);
  DGEN_HIP_TRY(hipMemsetAsync(c->d_arena, 0, bytes, c->s0));
  c->ops.assign(ops, ops + n_ops);
  c->max_frames = max_frames;
  c->configured = true;
  return run_static(c);
}

float* dgen_hip_host_memory(dgen_hip_ctx* c) { return c ? c->h_arena : nullptr; }

static int range_ok(dgen_hip_ctx* c, uint64_t off, uint64_t n, const char* what) {
  if (!c || !c->configured) return fail(DGEN_HIP_E_STATE, "%s: context not configured", what);
  if (off > c->floats || n > c->floats - off)
    return fail(DGEN_HIP_E_RANGE, "%s: [%llu, +%llu) outside arena of %llu floats", what,
                (unsigned long long)off, (unsigned long long)n, (unsigned long long)c->floats);
  return 0;
}

int dgen_hip_upload(dgen_hip_ctx* c, uint64_t off, uint64_t n) {
  int rc = range_ok(c, off, n, "upload");
  if (rc) return rc;
  if ((rc = set_device(c))) return rc;
  if (!n) return 0;
  DGEN_HIP_TRY(hipMemcpyAsync(c->d_arena + off, c->h_arena + off, n * sizeof(float), hipMemcpyHostToDevice, c->s0));
  DGEN_HIP_TRY(hipStreamSynchronize(c->s0));
  return 0;
}

int dgen_hip_download(dgen_hip_ctx* c, uint64_t off, uint64_t n) {
  int rc = range_ok(c, off, n, "download");
  if (rc) return rc;
  if ((rc = set_device(c))) return rc;
  if (!n) return 0;
  DGEN_HIP_TRY(hipMemcpyAsync(c->h_arena + off, c->d_arena + off, n * sizeof(float), hipMemcpyDeviceToHost, c->s0));
  DGEN_HIP_TRY(hipStreamSynchronize(c->s0));
  return 0;
}

int dgen_hip_zero(dgen_hip_ctx* c, uint64_t off, uint64_t n) {
  if (c && c->configured && n == 0 && off == 0) n = c->floats;
  int rc = range_ok(c, off, n, "zero");
  if (rc) return rc;
  if ((rc = set_device(c))) return rc;
  if (!n) return 0;
  DGEN_HIP_TRY(hipMemsetAsync(c->d_arena + off, 0, n * sizeof(float), c->s0));
  DGEN_HIP_TRY(hipStreamSynchronize(c->s0));
  return run_static(c);
}

// The frame-count argument of each per-run kernel class (index into
// op.arg; -1: no frame dimension) and whether the class runs any frame_count
// up to it (the first frame_count frames, as the reference's kernels loop
// over [0, frameCount) of cells sized for maxFrameCount) or only the frame
// count it was rendered for (its static tables, tiles and normalisation are
// laid out for that count).
struct FrameArg {
  int index;
  bool prefix;
};
static FrameArg frame_arg(uint32_t k) {
  switch (k) {
    case DGEN_HIP_K_PHASOR_CARRY: return {4, false};
    case DGEN_HIP_K_SYNTH_FWD:
    case DGEN_HIP_K_SYNTH_BWD: return {10, false};
    case DGEN_HIP_K_SPECTRAL_LOSS: return {4, false};
    case DGEN_HIP_K_SPECTRAL_GATHER: return {3, false};
    case DGEN_HIP_K_SYNTH_BWD_REDUCE: return {6, false};
    case DGEN_HIP_K_OSC_BANK: return {4, true};
    case DGEN_HIP_K_LERP_FRAMES: return {5, false};
    case DGEN_HIP_K_BIQUAD_CHUNK: return {5, false};
    case DGEN_HIP_K_BIQUAD_FWD: return {6, false};
    case DGEN_HIP_K_BIQUAD_ADJ_CHUNK: return {6, false};
    case DGEN_HIP_K_BIQUAD_BWD: return {8, false};
    case DGEN_HIP_K_STFT_FWD: return {7, false};
    case DGEN_HIP_K_STFT_BWD: return {5, false};
    case DGEN_HIP_K_MEMBRANE_FWD: return {6, false};
    case DGEN_HIP_K_MEMBRANE_BWD: return {9, false};
    case DGEN_HIP_K_STREAM_OSC_BANK: return {4, true};
    case DGEN_HIP_K_STREAM_BIQUAD: return {6, true};
    case DGEN_HIP_K_TEMPORAL_GRAD_SCAN: return {4, false};
    case DGEN_HIP_K_SWEPT_PHASOR: return {7, false};
    case DGEN_HIP_K_SVF_CHUNK: return {6, false};
    case DGEN_HIP_K_SVF_FWD:
    case DGEN_HIP_K_SVF_SEQ: return {10, false};
    case DGEN_HIP_K_STREAM_SVF: return {10, true};
    case DGEN_HIP_K_SVF_ADJ_CHUNK: return {8, false};
    case DGEN_HIP_K_SVF_BWD: return {11, false};
    case DGEN_HIP_K_UOP_BLOCK: return {7, true};
    default: return {-1, false};
  }
}

static int run_checks(dgen_hip_ctx* c, uint32_t frame_count) {
  if (!c || !c->configured) return fail(DGEN_HIP_E_STATE, "run: context not configured");
  if (frame_count == 0 || frame_count > c->max_frames)
    return fail(DGEN_HIP_E_RANGE, "run: frame_count %u outside [1, max_frames %u]", frame_count, c->max_frames);
  for (size_t i = 0; i < c->ops.size(); ++i) {
    const dgen_hip_op& op = c->ops[i];
    if (op.flags & DGEN_HIP_OP_STATIC) continue;
    const FrameArg fa = frame_arg(op.kernel);
    if (fa.index < 0) continue;
    const int64_t T = op.arg[fa.index];
    if (fa.prefix ? (int64_t)frame_count > T : (int64_t)frame_count != T)
      return fail(DGEN_HIP_E_RANGE, "run: op %zu (kernel %u) is rendered for %lld frames; frame_count %u %s", i,
                  op.kernel, (long long)T, frame_count, fa.prefix ? "exceeds it" : "must equal it");
  }
  return set_device(c);
}

// Static ops (temporality .static) depend only on their constant arguments;
// they run at configure and again after any zero() that may have cleared
// their outputs.
static int run_static(dgen_hip_ctx* c) {
  bool any = false;
  for (auto& op : c->ops) any |= (op.flags & DGEN_HIP_OP_STATIC) != 0;
  if (!any) return 0;
  int rc = enqueue(c, c->max_frames, true, nullptr);
  if (rc) return rc;
  DGEN_HIP_TRY(hipStreamSynchronize(c->s0));
  DGEN_HIP_TRY(hipStreamSynchronize(c->s1));
  return 0;
}

int dgen_hip_run_async(dgen_hip_ctx* c, uint32_t frame_count) {
  int rc = run_checks(c, frame_count);
  if (rc) return rc;
  rc = launch_run(c, frame_count);
  c->outputs_pending = rc == 0 && c->out_n != 0;
  return rc;
}

int dgen_hip_set_graphs(dgen_hip_ctx* c, int enable) {
  if (!c) return fail(DGEN_HIP_E_INVALID, "set_graphs: null context");
  int rc = set_device(c);
  if (rc) return rc;
  DGEN_HIP_TRY(hipStreamSynchronize(c->s0));
  DGEN_HIP_TRY(hipStreamSynchronize(c->s1));
  drop_graph(c);
  c->use_graphs = enable != 0;
  return 0;
}

// Wait for both streams (no output download).
static int sync_streams(dgen_hip_ctx* c) {
  int rc = set_device(c);
  if (rc) return rc;
  DGEN_HIP_TRY(hipStreamSynchronize(c->s0));
  DGEN_HIP_TRY(hipStreamSynchronize(c->s1));
  return 0;
}

int dgen_hip_sync(dgen_hip_ctx* c) {
  if (!c) return fail(DGEN_HIP_E_INVALID, "sync: null context");
  int rc = sync_streams(c);
  if (rc) return rc;
  // the declared outputs of a dgen_hip_run_async become host-visible here, as
  // the reference's shared-storage outputs buffer is after run()
  // (MetalRuntime.swift:232, 334-337)
  if (c->outputs_pending) {
    c->outputs_pending = false;
    if (c->out_n) return dgen_hip_download(c, c->out_off, c->out_n);
  }
  return 0;
}

int dgen_hip_run(dgen_hip_ctx* c, uint32_t frame_count) {
  int rc = dgen_hip_run_async(c, frame_count);
  if (rc) {
    if (c) (void)sync_streams(c);
    return rc;
  }
  return dgen_hip_sync(c);
}

int dgen_hip_set_outputs(dgen_hip_ctx* c, uint64_t off, uint64_t n) {
  int rc = range_ok(c, off, n, "set_outputs");
  if (rc) return rc;
  c->out_off = off;
  c->out_n = n;
  return 0;
}

float* dgen_hip_host_outputs(dgen_hip_ctx* c, uint64_t* n_out) {
  if (n_out) *n_out = (c && c->configured) ? c->out_n : 0;
  if (!c || !c->configured || !c->out_n) return nullptr;
  return c->h_arena + c->out_off;
}

int dgen_hip_set_process_ports(dgen_hip_ctx* c, uint32_t n_in, const uint64_t* in_cells, const uint32_t* in_strides,
                               uint32_t n_out, const uint64_t* out_cells, const uint32_t* out_strides) {
  if (!c || !c->configured) return fail(DGEN_HIP_E_STATE, "set_process_ports: context not configured");
  if ((n_in && (!in_cells || !in_strides)) || (n_out && (!out_cells || !out_strides)))
    return fail(DGEN_HIP_E_INVALID, "set_process_ports: null port arrays");
  auto check = [&](const uint64_t* cells, const uint32_t* strides, uint32_t n, const char* what) -> int {
    for (uint32_t i = 0; i < n; ++i) {
      if (strides[i] == 0)
        return fail(DGEN_HIP_E_INVALID, "set_process_ports: %s channel %u has stride 0", what, i);
      const uint64_t last = cells[i] + (uint64_t)(c->max_frames - 1) * strides[i];
      if (cells[i] >= c->floats || last >= c->floats)
        return fail(DGEN_HIP_E_RANGE, "set_process_ports: %s channel %u ([%llu, %llu] over %u frames) outside arena "
                    "of %llu floats", what, i, (unsigned long long)cells[i], (unsigned long long)last, c->max_frames,
                    (unsigned long long)c->floats);
    }
    return 0;
  };
  int rc = check(in_cells, in_strides, n_in, "input");
  if (!rc) rc = check(out_cells, out_strides, n_out, "output");
  if (rc) return rc;
  // input channels must not share a cell: a call writes each input cell from
  // exactly one channel (and process_v1 relies on it to tell whether the
  // ports fill their span)
  if (n_in > 1) {
    uint64_t lo = UINT64_MAX, hi = 0;
    for (uint32_t i = 0; i < n_in; ++i) {
      lo = std::min(lo, in_cells[i]);
      hi = std::max(hi, in_cells[i] + (uint64_t)(c->max_frames - 1) * in_strides[i] + 1);
    }
    std::vector<uint8_t> used(hi - lo, 0);
    for (uint32_t i = 0; i < n_in; ++i)
      for (uint32_t f = 0; f < c->max_frames; ++f) {
        uint8_t& u = used[in_cells[i] + (uint64_t)f * in_strides[i] - lo];
        if (u) return fail(DGEN_HIP_E_INVALID, "set_process_ports: input channel %u frame %u shares cell %llu with "
                           "another input channel", i, f, (unsigned long long)(in_cells[i] + (uint64_t)f * in_strides[i]));
        u = 1;
      }
  }
  c->in_cell.assign(in_cells, in_cells + n_in);
  c->in_stride.assign(in_strides, in_strides + n_in);
  c->out_cell.assign(out_cells, out_cells + n_out);
  c->out_stride.assign(out_strides, out_strides + n_out);
  return 0;
}

// Smallest cell range covering `n` frames of every channel of a port list.
static void port_span(const std::vector<uint64_t>& cells, const std::vector<uint32_t>& strides, uint32_t n,
                      uint64_t* lo, uint64_t* hi) {
  *lo = UINT64_MAX;
  *hi = 0;
  for (size_t i = 0; i < cells.size(); ++i) {
    *lo = std::min(*lo, cells[i]);
    *hi = std::max(*hi, cells[i] + (uint64_t)(n - 1) * strides[i] + 1);
  }
}

int dgen_hip_process_v1(dgen_hip_ctx* c, const float* const* inputs, float* const* outputs, uint32_t frame_count,
                        const dgen_hip_process_context_v1* context) {
  if (!c || !c->configured) return fail(DGEN_HIP_E_STATE, "process_v1: context not configured");
  float sr = 0.f;
  uint32_t flags = 0;
  if (context) {
    if (context->abi_version != DGEN_HIP_ABI_VERSION || context->struct_size < sizeof(dgen_hip_process_context_v1))
      return fail(DGEN_HIP_E_INVALID, "process_v1: context abi %u size %u (expected %d, >= %zu)",
                  context->abi_version, context->struct_size, DGEN_HIP_ABI_VERSION,
                  sizeof(dgen_hip_process_context_v1));
    sr = context->sample_rate;
    flags = context->flags;
    if (!(sr == 0.f || (sr >= 1.f && sr <= 1e7f)))
      return fail(DGEN_HIP_E_INVALID, "process_v1: sample rate %g Hz outside [1, 1e7] (or 0)", (double)sr);
  }
  int rc = run_checks(c, frame_count);
  if (rc) return rc;
  if (!c->in_cell.empty() && !inputs) return fail(DGEN_HIP_E_INVALID, "process_v1: null inputs");
  if (!c->out_cell.empty() && !outputs) return fail(DGEN_HIP_E_INVALID, "process_v1: null outputs");
  for (size_t i = 0; i < c->in_cell.size(); ++i)
    if (!inputs[i]) return fail(DGEN_HIP_E_INVALID, "process_v1: input channel %zu is null", i);
  for (size_t i = 0; i < c->out_cell.size(); ++i)
    if (!outputs[i]) return fail(DGEN_HIP_E_INVALID, "process_v1: output channel %zu is null", i);
  // inputs -> host mirror -> device, one copy over the ports' span.  When the
  // ports do not fill their span (the span holds cells of other data, e.g.
  // state the device carries between calls), the span is refreshed from the
  // device first, so the copy writes those cells back unchanged.
  if (!c->in_cell.empty()) {
    uint64_t lo, hi;
    port_span(c->in_cell, c->in_stride, frame_count, &lo, &hi);
    if ((uint64_t)c->in_cell.size() * frame_count != hi - lo && (rc = dgen_hip_download(c, lo, hi - lo))) return rc;
    for (size_t i = 0; i < c->in_cell.size(); ++i) {
      float* dst = c->h_arena + c->in_cell[i];
      const uint32_t st = c->in_stride[i];
      for (uint32_t f = 0; f < frame_count; ++f) dst[(size_t)f * st] = inputs[i][f];
    }
    if ((rc = dgen_hip_upload(c, lo, hi - lo))) return rc;
  }
  // the run, eagerly enqueued, at the call's host rate and reset flag
  const float saved_sr = c->host_sr;
  c->host_sr = sr;
  c->reset_next = (flags & DGEN_HIP_PROCESS_RESET) != 0;
  rc = enqueue(c, frame_count, false, nullptr);
  c->host_sr = saved_sr;
  c->reset_next = false;
  const int rc2 = dgen_hip_sync(c);
  if (rc || rc2) return rc ? rc : rc2;
  if (!c->out_cell.empty()) {
    uint64_t lo, hi;
    port_span(c->out_cell, c->out_stride, frame_count, &lo, &hi);
    if ((rc = dgen_hip_download(c, lo, hi - lo))) return rc;
    for (size_t i = 0; i < c->out_cell.size(); ++i) {
      const float* src = c->h_arena + c->out_cell[i];
      const uint32_t st = c->out_stride[i];
      for (uint32_t f = 0; f < frame_count; ++f) outputs[i][f] = src[(size_t)f * st];
    }
  }
  return 0;
}

int dgen_hip_set_sample_rate(dgen_hip_ctx* c, float sample_rate) {
  if (!c) return fail(DGEN_HIP_E_INVALID, "set_sample_rate: null context");
  // 0 restores each op's rendered rate; otherwise a rate the phase kernels'
  // reciprocal-product division is exact for (normal quotients on [1, 1e7] Hz)
  if (!(sample_rate == 0.f || (sample_rate >= 1.f && sample_rate <= 1e7f)))
    return fail(DGEN_HIP_E_INVALID, "set_sample_rate: %g Hz outside [1, 1e7] (or 0)", (double)sample_rate);
  int rc = set_device(c);
  if (rc) return rc;
  DGEN_HIP_TRY(hipStreamSynchronize(c->s0));
  DGEN_HIP_TRY(hipStreamSynchronize(c->s1));
  if (sample_rate != c->host_sr) drop_graph(c);  // captured launches hold the old rate
  c->host_sr = sample_rate;
  return 0;
}

int dgen_hip_profile(dgen_hip_ctx* c, uint32_t frame_count, dgen_hip_kernel_time* out, size_t cap, size_t* n_out) {
  int rc = run_checks(c, frame_count);
  if (rc) return rc;
  std::vector<hipEvent_t> evs(2 * c->ops.size(), nullptr);
  for (auto& e : evs) DGEN_HIP_TRY(hipEventCreate(&e));
  rc = enqueue(c, frame_count, false, &evs);
  int rc2 = dgen_hip_sync(c);
  size_t n = 0;
  if (!rc && !rc2) {
    for (size_t i = 0; i < c->ops.size(); ++i) {
      if (c->ops[i].flags & DGEN_HIP_OP_STATIC) continue;
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, evs[2 * i], evs[2 * i + 1]) != hipSuccess) ms = -1.f;
      if (out && n < cap) out[n] = dgen_hip_kernel_time{(uint32_t)i, c->ops[i].kernel, ms};
      ++n;
    }
  }
  for (auto& e : evs) (void)hipEventDestroy(e);
  if (n_out) *n_out = n;
  return rc ? rc : rc2;
}

int dgen_hip_time_runs(dgen_hip_ctx* c, uint32_t frame_count, int warmup, int iters, double* ms_out) {
  if (!ms_out || iters <= 0 || warmup < 0) return fail(DGEN_HIP_E_INVALID, "time_runs: bad arguments");
  int rc = run_checks(c, frame_count);
  if (rc) return rc;
  for (int i = 0; i < warmup; ++i)
    if ((rc = launch_run(c, frame_count))) return rc;
  if ((rc = dgen_hip_sync(c))) return rc;
  hipEvent_t a, b;
  DGEN_HIP_TRY(hipEventCreate(&a));
  DGEN_HIP_TRY(hipEventCreate(&b));
  DGEN_HIP_TRY(hipEventRecord(a, c->s0));
  for (int i = 0; i < iters && !rc; ++i) rc = launch_run(c, frame_count);
  DGEN_HIP_TRY(hipEventRecord(b, c->s0));
  int rc2 = dgen_hip_sync(c);
  float ms = 0.f;
  if (!rc && !rc2) DGEN_HIP_TRY(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  *ms_out = ms;
  return rc ? rc : rc2;
}

int dgen_hip_run_op(dgen_hip_ctx* c, uint32_t frame_count, uint32_t op_index) {
  int rc = run_checks(c, frame_count);
  if (rc) return rc;
  if (op_index >= c->ops.size()) return fail(DGEN_HIP_E_INVALID, "run_op: op %u of %zu", op_index, c->ops.size());
  const dgen_hip_op& op = c->ops[op_index];
  hipStream_t s = (op.flags & DGEN_HIP_OP_SIDE) ? c->s1 : c->s0;
  rc = launcher_for(op.kernel)(make_launch(c, s, frame_count, false), op);
  int rc2 = dgen_hip_sync(c);
  return rc ? rc : rc2;
}

int dgen_hip_time_op(dgen_hip_ctx* c, uint32_t frame_count, uint32_t op_index, int iters, double* ms_out) {
  if (!ms_out || iters <= 0) return fail(DGEN_HIP_E_INVALID, "time_op: bad arguments");
  int rc = run_checks(c, frame_count);
  if (rc) return rc;
  if (op_index >= c->ops.size() || (c->ops[op_index].flags & DGEN_HIP_OP_STATIC))
    return fail(DGEN_HIP_E_INVALID, "time_op: op %u is not a per-run op", op_index);
  std::vector<hipEvent_t> evs(2 * c->ops.size(), nullptr);
  for (auto& e : evs) DGEN_HIP_TRY(hipEventCreate(&e));
  double total = 0.0;
  for (int it = 0; it < iters && !rc; ++it) {
    rc = enqueue(c, frame_count, false, &evs);
    int rc2 = dgen_hip_sync(c);
    if (!rc) rc = rc2;
    float ms = 0.f;
    if (!rc && hipEventElapsedTime(&ms, evs[2 * op_index], evs[2 * op_index + 1]) != hipSuccess)
      rc = fail(DGEN_HIP_E_DEVICE, "time_op: hipEventElapsedTime failed");
    total += ms;
  }
  for (auto& e : evs) (void)hipEventDestroy(e);
  *ms_out = total / iters;
  return rc;
}

int dgen_hip_time_op_alone(dgen_hip_ctx* c, uint32_t frame_count, uint32_t op_index, int iters, double* ms_out) {
  if (!ms_out || iters <= 0) return fail(DGEN_HIP_E_INVALID, "time_op_alone: bad arguments");
  int rc = run_checks(c, frame_count);
  if (rc) return rc;
  if (op_index >= c->ops.size() || (c->ops[op_index].flags & DGEN_HIP_OP_STATIC))
    return fail(DGEN_HIP_E_INVALID, "time_op_alone: op %u is not a per-run op", op_index);
  rc = dgen_hip_sync(c);
  if (rc) return rc;
  const dgen_hip_op& op = c->ops[op_index];
  const Launch L = make_launch(c, c->s0, frame_count, false);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  DGEN_HIP_TRY(hipEventCreate(&e0));
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return fail(DGEN_HIP_E_DEVICE, "time_op_alone: hipEventCreate failed");
  }
  rc = launcher_for(op.kernel)(L, op);
  if (!rc && hipEventRecord(e0, c->s0) != hipSuccess) rc = fail(DGEN_HIP_E_DEVICE, "time_op_alone: event record");
  for (int it = 0; it < iters && !rc; ++it) rc = launcher_for(op.kernel)(L, op);
  if (!rc && hipEventRecord(e1, c->s0) != hipSuccess) rc = fail(DGEN_HIP_E_DEVICE, "time_op_alone: event record");
  const int rc2 = dgen_hip_sync(c);
  if (!rc) rc = rc2;
  float ms = 0.f;
  if (!rc && hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
    rc = fail(DGEN_HIP_E_DEVICE, "time_op_alone: hipEventElapsedTime failed");
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *ms_out = rc ? 0.0 : (double)ms / iters;
  return rc;
}

// ---- generic UOp blocks: hiprtc compile with a per-process cache ---------
namespace {
std::mutex g_rtc_mu;
std::vector<std::pair<std::string, std::vector<char>>> g_rtc_cache;  // source -> code object
}  // namespace

// Compile HIP C++ for gfx950: packed fp32 off, as every kernel here, and no
// contraction of a*b+c into fma, so each UOp rounds as the reference's fp32
// node does (a contracted (f/sr)*n - floor(...) moves a phase by half an ulp
// of the product: up to 2.4e-4 revolutions at n = 65536).
static int rtc_compile(const std::string& src, std::vector<char>& code) {
  {
    std::lock_guard<std::mutex> lk(g_rtc_mu);
    for (const auto& e : g_rtc_cache)
      if (e.first == src) {
        code = e.second;
        return 0;
      }
  }
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "dgen_blocks.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    return fail(DGEN_HIP_E_INVALID, "blocks: hiprtcCreateProgram failed");
  const char* opts[] = {"--offload-arch=gfx950", "-O3",           "-ffp-contract=off", "-Xclang",
                        "-target-feature",       "-Xclang",       "-packed-fp32-ops"};
  const hiprtcResult r = hiprtcCompileProgram(prog, 7, opts);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n + 1, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    return fail(DGEN_HIP_E_INVALID, "blocks: compile failed: %s", log.c_str());
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  code.assign(n, 0);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  std::lock_guard<std::mutex> lk(g_rtc_mu);
  g_rtc_cache.emplace_back(src, code);
  return 0;
}

int dgen_hip_render_blocks(const dgen_hip_block* blocks, uint32_t n, int compile, char* buf, size_t cap, size_t* len) {
  std::string src;
  int rc = render_blocks(blocks, n, src);
  if (rc) return rc;
  if (len) *len = src.size();
  if (buf && cap) {
    const size_t k = std::min(cap - 1, src.size());
    std::memcpy(buf, src.data(), k);
    buf[k] = '\0';
  }
  if (compile) {
    std::vector<char> code;
    if ((rc = rtc_compile(src, code))) return rc;
  }
  return 0;
}

int dgen_hip_set_blocks(dgen_hip_ctx* c, const dgen_hip_block* blocks, uint32_t n) {
  if (!c) return fail(DGEN_HIP_E_INVALID, "set_blocks: null context");
  std::string src;
  int rc = render_blocks(blocks, n, src);
  if (rc) return rc;
  std::vector<char> code;
  if (n && (rc = rtc_compile(src, code))) return rc;
  if ((rc = set_device(c))) return rc;
  DGEN_HIP_TRY(hipStreamSynchronize(c->s0));
  DGEN_HIP_TRY(hipStreamSynchronize(c->s1));
  drop_graph(c);
  if (c->blk_module) {
    (void)hipModuleUnload(c->blk_module);
    c->blk_module = nullptr;
  }
  c->blocks.clear();
  if (!n) return 0;
  DGEN_HIP_TRY(hipModuleLoadData(&c->blk_module, code.data()));
  c->blocks.resize(n);
  for (uint32_t i = 0; i < n; ++i) {
    BlockInfo& b = c->blocks[i];
    const std::string name = "dgen_block_" + std::to_string(i);
    DGEN_HIP_TRY(hipModuleGetFunction(&b.fn, c->blk_module, name.c_str()));
    b.dispatch = blocks[i].dispatch;
    b.n = blocks[i].dispatch_n;
    b.frame_order = blocks[i].frame_order;
    b.max_cell = block_max_cell(blocks[i]);
  }
  return 0;
}

// ---- the reference-named process-function exports (dgen_process_v1.h) ----
// One bound schedule per process, as the reference loads one compiled graph
// per process-function library.  The graph's memory range of the arena is
// copied from the caller's state block before each block and back after it,
// so every instance's carried state lives in its own block.
namespace {
std::mutex g_proc_mu;
dgen_hip_ctx* g_proc_ctx = nullptr;
uint64_t g_proc_off = 0, g_proc_n = 0;
}  // namespace

static void process_unbind_if(dgen_hip_ctx* c) {
  std::lock_guard<std::mutex> lk(g_proc_mu);
  if (g_proc_ctx == c) {
    g_proc_ctx = nullptr;
    g_proc_off = g_proc_n = 0;
  }
}

int dgen_hip_process_bind(dgen_hip_ctx* c, uint64_t off, uint64_t n) {
  std::lock_guard<std::mutex> lk(g_proc_mu);
  if (!c) {
    g_proc_ctx = nullptr;
    g_proc_off = g_proc_n = 0;
    return 0;
  }
  if (!c->configured) return fail(DGEN_HIP_E_STATE, "process_bind: context not configured");
  if (c->in_cell.empty() && c->out_cell.empty())
    return fail(DGEN_HIP_E_STATE, "process_bind: the context has no process ports (dgen_hip_set_process_ports)");
  if (n == 0 || off > c->floats || n > c->floats - off)
    return fail(DGEN_HIP_E_RANGE, "process_bind: memory [%llu, +%llu) outside the arena of %llu floats",
                (unsigned long long)off, (unsigned long long)n, (unsigned long long)c->floats);
  g_proc_ctx = c;
  g_proc_off = off;
  g_proc_n = n;
  return 0;
}

uint64_t dgen_hip_process_memory_size(void) {
  std::lock_guard<std::mutex> lk(g_proc_mu);
  return g_proc_ctx ? std::max<uint64_t>(g_proc_n, 1024) : 0;
}

void dgen_process_v1(const float* const* inputs, float* const* outputs, uint32_t frame_count, void* state,
                     const DGenProcessContextV1* context, const DGenHostServicesV1* host) {
  (void)host;
  std::lock_guard<std::mutex> lk(g_proc_mu);
  dgen_hip_ctx* c = g_proc_ctx;
  // silence on failure: every output channel the bound ports name, for the
  // frames the call asked for
  auto silence = [&]() {
    if (!c || !outputs) return;
    for (size_t i = 0; i < c->out_cell.size(); ++i)
      if (outputs[i]) std::memset(outputs[i], 0, (size_t)frame_count * sizeof(float));
  };
  if (!c) {
    fail(DGEN_HIP_E_STATE, "dgen_process_v1: no schedule bound (dgen_hip_process_bind)");
    return;
  }
  if (!state) {
    fail(DGEN_HIP_E_INVALID, "dgen_process_v1: null state block");
    silence();
    return;
  }
  // the reference's reading of the context (CRenderer.swift:357-359): its
  // rate counts only for a v1 struct of full size; otherwise the graph's own
  dgen_hip_process_context_v1 pc{DGEN_HIP_ABI_VERSION, sizeof(dgen_hip_process_context_v1), 0.f, 0u};
  if (context && context->abi_version == DGEN_ABI_VERSION_V1 && context->struct_size >= sizeof(DGenProcessContextV1))
    pc.sample_rate = context->sample_rate;
  float* blk = static_cast<float*>(state);
  int rc = run_checks(c, frame_count);
  if (!rc) {
    std::memcpy(c->h_arena + g_proc_off, blk, g_proc_n * sizeof(float));
    rc = dgen_hip_upload(c, g_proc_off, g_proc_n);
  }
  if (!rc) rc = dgen_hip_process_v1(c, inputs, outputs, frame_count, &pc);
  if (!rc) rc = dgen_hip_download(c, g_proc_off, g_proc_n);
  if (rc) {
    silence();
    return;
  }
  std::memcpy(blk, c->h_arena + g_proc_off, g_proc_n * sizeof(float));
}

void dgen_set_param_value_v1(int32_t cell_id, float value) {
  (void)cell_id;
  (void)value;
}

}  // extern "C"
