// Generic lowering of DGen UOp blocks to HIP C++ (the MetalRenderer's
// prepareSchedule + render + emit, Sources/DGen/Renderer/MetalRenderer.swift:
// 787-938, 940-1120, 1316-1720), compiled at configure time with hiprtc.
//
// A block is the compiler's BlockUOps (Renderer.swift:3-24): its UOps, frame
// order, temporality and dispatch mode.  Each block becomes one kernel
// `dgen_block_<i>(memory, t, outputs, inputs, frameCount, hostSampleRate,
// memFloats, tapeFloats, outFloats, inFloats)`:
//   - the range guard and the renderer's frame loop of the dispatch mode
//     (singleThreaded / fixedWithFrameLoop / sequential perFrameScaled loop
//     the frames on their threads; perFrame* runs one frame per thread), and
//     the hop check of a hop-based block;
//   - cells are float offsets into `memory` (the arena), tape globals live in
//     `t[slot * frameCount + frame]` (static globals at frame 0), outputs in
//     `outputs[channel * frameCount + frame]`, inputs likewise;
//   - every index computed at run time into memory, tape, outputs and inputs
//     is clamped into its array (an out-of-range index reads or writes the
//     array's last element instead of faulting), and output stores map
//     non-finite values to 0, as the C backend's do (dgen_runtime.h:72-85).
// GEMM dispatch modes are not lowered here (GEMM blocks are the MFMA GEMM
// class, DGEN_HIP_K_GEMM), nor the C-only vDSP calls.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "internal.h"

namespace dgen {

namespace {

// fp32 value as an exact hexadecimal float literal
std::string flit(float v) {
  if (std::isnan(v)) return "__builtin_nanf(\"\")";
  if (std::isinf(v)) return v > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
  char b[64];
  snprintf(b, sizeof b, "%af", (double)v);
  return b;
}

struct Renderer {
  const dgen_hip_block& blk;
  int index;
  const std::set<int>& static_slots;
  std::string out;
  std::string err;
  int indent = 1;
  // per-kernel state (MetalRenderer.render)
  std::set<int> int_vars;       // variables declared int
  std::set<int> pr_vars;        // parallel-range loop variables (_pr<id>)
  std::set<int> declared;       // locals declared so far
  bool frame_override = false;  // setFrameIndex seen
  int scale = 0;                // threadCountScale (perFrameScaled n)
  bool parallel = false;        // frameOrder == parallel

  Renderer(const dgen_hip_block& b, int i, const std::set<int>& ss) : blk(b), index(i), static_slots(ss) {}

  void line(const std::string& s) {
    out.append((size_t)indent * 2, ' ');
    out += s;
    out += '\n';
  }
  bool bad(const char* fmt, ...) __attribute__((format(printf, 2, 3))) {
    char b[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(b, sizeof b, fmt, ap);
    va_end(ap);
    if (err.empty()) err = b;
    return false;
  }

  // the frame index the tape, outputs and inputs use
  std::string base_idx() const { return parallel ? "id" : "i"; }
  std::string frame_idx() const {
    if (frame_override) return "_frameIndex";
    if (scale > 0) return "(" + base_idx() + " / " + std::to_string(scale) + "u)";
    return base_idx();
  }
  std::string tape(int slot) const {
    const std::string idx = static_slots.count(slot) ? std::string("0u") : frame_idx();
    return "t[DG_T((unsigned long long)" + std::to_string(slot) + "u * frameCount + " + idx + ")]";
  }

  bool lazy(const dgen_hip_lazy& l, bool as_int, std::string& s) {
    switch (l.kind) {
      case DGEN_HIP_LAZY_CONST:
        if (as_int) {
          char b[32];
          snprintf(b, sizeof b, "%lld", (long long)l.value);
          s = b;
        } else {
          s = flit(l.value);
        }
        return true;
      case DGEN_HIP_LAZY_VAR:
        if (pr_vars.count(l.id)) s = "_pr" + std::to_string(l.id);
        else s = "t" + std::to_string(l.id);
        return true;
      case DGEN_HIP_LAZY_GLOBAL:
        if (l.id < 0) return bad("block %d: tape slot %d", index, l.id);
        s = tape(l.id);
        return true;
      case DGEN_HIP_LAZY_FRAME_COUNT:
        s = "frameCount";
        return true;
      default:
        return bad("block %d: empty operand", index);
    }
  }
  bool g(const dgen_hip_lazy& l, std::string& s) { return lazy(l, false, s); }
  bool is_int(const dgen_hip_lazy& l) const { return l.kind == DGEN_HIP_LAZY_VAR && int_vars.count(l.id); }

  // declare-or-assign of the UOp's value (MetalRenderer.emitAssign)
  bool assign(const dgen_hip_uop& u, const std::string& expr) {
    const dgen_hip_lazy& v = u.value;
    if (v.kind == DGEN_HIP_LAZY_GLOBAL) {
      line(tape(v.id) + " = " + expr + ";");
      return true;
    }
    if (v.kind != DGEN_HIP_LAZY_VAR) return bad("block %d: op %d assigns to a non-variable", index, u.op);
    const std::string name = "t" + std::to_string(v.id);
    if (u.int_typed) int_vars.insert(v.id);
    else int_vars.erase(v.id);
    line(std::string(u.int_typed ? "int " : "float ") + name + " = " + expr + ";");
    declared.insert(v.id);
    return true;
  }

  std::string mem(int64_t cell) const { return "memory[" + std::to_string(cell) + "]"; }
  std::string mem_off(int64_t cell, const std::string& off) const {
    return "memory[DG_M((long long)" + std::to_string(cell) + " + (long long)(" + off + "))]";
  }

  bool emit(const dgen_hip_uop& u) {
    std::string a, b, c;
    auto need = [&](int n) -> bool {
      if (n >= 1 && !g(u.a, a)) return false;
      if (n >= 2 && !g(u.b, b)) return false;
      if (n >= 3 && !g(u.c, c)) return false;
      return true;
    };
    auto ia = [&](const dgen_hip_lazy& l, std::string& s) { return lazy(l, u.int_typed != 0, s); };
    switch (u.op) {
      case DGEN_HIP_UOP_ADD:
      case DGEN_HIP_UOP_SUB:
      case DGEN_HIP_UOP_MUL: {
        if (!ia(u.a, a) || !ia(u.b, b)) return false;
        const char* o = u.op == DGEN_HIP_UOP_ADD ? " + " : (u.op == DGEN_HIP_UOP_SUB ? " - " : " * ");
        return assign(u, a + o + b);
      }
      case DGEN_HIP_UOP_DIV:
        if (!ia(u.a, a) || !ia(u.b, b)) return false;
        return assign(u, a + " / " + b);
      case DGEN_HIP_UOP_MOD:
        if (u.int_typed) {
          if (!ia(u.a, a) || !ia(u.b, b)) return false;
          return assign(u, a + " % " + b);
        }
        if (!need(2)) return false;
        if (u.b.kind == DGEN_HIP_LAZY_CONST && u.b.value == 1.0f) return assign(u, "(" + a + " - floorf(" + a + "))");
        return assign(u, "fmodf(" + a + ", " + b + ")");
      case DGEN_HIP_UOP_POW:
        if (!need(2)) return false;
        return assign(u, "powf(" + a + ", " + b + ")");
      case DGEN_HIP_UOP_MIN:
        if (!need(2)) return false;
        return assign(u, "fminf(" + a + ", " + b + ")");
      case DGEN_HIP_UOP_MAX:
        if (!need(2)) return false;
        return assign(u, "fmaxf(" + a + ", " + b + ")");
      case DGEN_HIP_UOP_ATAN2:
        if (!need(2)) return false;
        return assign(u, "atan2f(" + a + ", " + b + ")");
      case DGEN_HIP_UOP_ABS:
      case DGEN_HIP_UOP_SIGN:
      case DGEN_HIP_UOP_SIN:
      case DGEN_HIP_UOP_COS:
      case DGEN_HIP_UOP_TAN:
      case DGEN_HIP_UOP_ATAN:
      case DGEN_HIP_UOP_TANH:
      case DGEN_HIP_UOP_EXP:
      case DGEN_HIP_UOP_LOG:
      case DGEN_HIP_UOP_LOG10:
      case DGEN_HIP_UOP_SQRT:
      case DGEN_HIP_UOP_FLOOR:
      case DGEN_HIP_UOP_CEIL:
      case DGEN_HIP_UOP_ROUND: {
        if (!need(1)) return false;
        static const std::map<int, const char*> fn = {
            {DGEN_HIP_UOP_ABS, "fabsf"},   {DGEN_HIP_UOP_SIGN, "dg_sign"}, {DGEN_HIP_UOP_SIN, "sinf"},
            {DGEN_HIP_UOP_COS, "cosf"},    {DGEN_HIP_UOP_TAN, "tanf"},     {DGEN_HIP_UOP_ATAN, "atanf"},
            {DGEN_HIP_UOP_TANH, "tanhf"},  {DGEN_HIP_UOP_EXP, "expf"},     {DGEN_HIP_UOP_LOG, "logf"},
            {DGEN_HIP_UOP_LOG10, "log10f"}, {DGEN_HIP_UOP_SQRT, "sqrtf"},  {DGEN_HIP_UOP_FLOOR, "floorf"},
            {DGEN_HIP_UOP_CEIL, "ceilf"},  {DGEN_HIP_UOP_ROUND, "roundf"}};
        return assign(u, std::string(fn.at(u.op)) + "(" + a + ")");
      }
      case DGEN_HIP_UOP_GT:
      case DGEN_HIP_UOP_GTE:
      case DGEN_HIP_UOP_LTE:
      case DGEN_HIP_UOP_LT:
      case DGEN_HIP_UOP_EQ: {
        if (!need(2)) return false;
        static const std::map<int, const char*> op = {{DGEN_HIP_UOP_GT, " > "},
                                                      {DGEN_HIP_UOP_GTE, " >= "},
                                                      {DGEN_HIP_UOP_LTE, " <= "},
                                                      {DGEN_HIP_UOP_LT, " < "},
                                                      {DGEN_HIP_UOP_EQ, " == "}};
        return assign(u, "(" + a + op.at(u.op) + b + ")");
      }
      // logical ops on 0/1 floats (CRenderer.swift:864-885)
      case DGEN_HIP_UOP_AND:
        if (!need(2)) return false;
        return assign(u, "(((" + a + ") != 0.0f && (" + b + ") != 0.0f) ? 1.0f : 0.0f)");
      case DGEN_HIP_UOP_OR:
        if (!need(2)) return false;
        return assign(u, "(((" + a + ") != 0.0f || (" + b + ") != 0.0f) ? 1.0f : 0.0f)");
      case DGEN_HIP_UOP_XOR:
        if (!need(2)) return false;
        return assign(u, "((((" + a + ") != 0.0f) != ((" + b + ") != 0.0f)) ? 1.0f : 0.0f)");
      case DGEN_HIP_UOP_GSWITCH: {
        // select(b, a, cond > 0) (MetalRenderer.swift:1453-1458)
        if (!need(3)) return false;
        const std::string av = is_int(u.b) ? "(float)" + b : b, bv = is_int(u.c) ? "(float)" + c : c;
        return assign(u, "((" + a + ") > 0.0f ? " + av + " : " + bv + ")");
      }
      case DGEN_HIP_UOP_SELECTOR: {
        // mode <= 0: 0; mode <= i+1: options[i]; beyond the last: 0
        // (MetalRenderer.swift:1466-1478)
        if (!need(1)) return false;
        if (u.n_list && !u.list) return bad("block %d: selector without options", index);
        std::string e = "0.0f";
        for (int i = (int)u.n_list - 1; i >= 0; --i) {
          std::string o;
          if (!g(u.list[i], o)) return false;
          e = "((" + a + ") <= " + flit((float)(i + 1)) + " ? " + o + " : " + e + ")";
        }
        return assign(u, "((" + a + ") <= 0.0f ? 0.0f : " + e + ")");
      }
      case DGEN_HIP_UOP_IDENTITY:
      case DGEN_HIP_UOP_DECLARE_VAR:
      case DGEN_HIP_UOP_BROADCAST_SCALAR:
        if (!ia(u.a, a)) return false;
        return assign(u, a);
      case DGEN_HIP_UOP_CAST:
        if (!need(1)) return false;
        return assign(u, std::string(u.imm[0] ? "(int)(" : "(float)(") + a + ")");
      case DGEN_HIP_UOP_MUTATE: {
        if (!g(u.b, b)) return false;
        if (u.a.kind == DGEN_HIP_LAZY_GLOBAL) {
          line(tape(u.a.id) + " = " + b + ";");
          return true;
        }
        if (!g(u.a, a)) return false;
        line(a + " = " + b + ";");
        return true;
      }
      // ---- memory cells
      case DGEN_HIP_UOP_LOAD:
        return assign(u, mem(u.imm[0]));
      case DGEN_HIP_UOP_STORE:
        if (!need(1)) return false;
        line(mem(u.imm[0]) + " = " + a + ";");
        return true;
      case DGEN_HIP_UOP_DELAY1:
        // the previous frame's value, then this frame's (MetalRenderer.swift:1460-1464)
        if (!need(1)) return false;
        if (!assign(u, mem(u.imm[0]))) return false;
        line(mem(u.imm[0]) + " = " + a + ";");
        return true;
      case DGEN_HIP_UOP_NOISE: {
        // xorshift32 on the cell's bits (MetalRenderer.swift:1387-1399)
        const std::string m = mem(u.imm[0]);
        line("{");
        line("  unsigned _s = __float_as_uint(" + m + ");");
        line("  if (_s == 0u) _s = 1u;");
        line("  _s ^= _s << 13; _s ^= _s >> 17; _s ^= _s << 5;");
        line("  " + m + " = __uint_as_float(_s);");
        line("  _noise = (float)_s / 4294967296.0f;");
        line("}");
        return assign(u, "_noise");
      }
      case DGEN_HIP_UOP_MEMORY_READ:
      case DGEN_HIP_UOP_SIMD_BROADCAST_LOAD:
        if (!need(1)) return false;
        return assign(u, mem_off(u.imm[0], a));
      case DGEN_HIP_UOP_MEMORY_WRITE:
        if (!need(2)) return false;
        line(mem_off(u.imm[0], a) + " = " + b + ";");
        return true;
      case DGEN_HIP_UOP_MEMORY_ACCUMULATE:
        if (!need(2)) return false;
        line("atomicAdd(&" + mem_off(u.imm[0], a) + ", " + b + ");");
        return true;
      case DGEN_HIP_UOP_LOAD_TAPE: {
        // a bounded tape read of another frame (MetalRenderer.swift:1506-1510)
        if (u.a.kind != DGEN_HIP_LAZY_GLOBAL) return bad("block %d: loadTape of a non-global", index);
        if (!g(u.b, b)) return false;
        const std::string slot = std::to_string(u.a.id);
        return assign(u, "((" + b + ") < 0 || (" + b + ") >= (float)frameCount ? 0.0f : t[DG_T((unsigned long long)" +
                             slot + "u * frameCount + (unsigned long long)(int)(" + b + "))])");
      }
      // ---- control flow
      case DGEN_HIP_UOP_BEGIN_IF:
        if (!need(1)) return false;
        line("if (" + a + ") {");
        ++indent;
        return true;
      case DGEN_HIP_UOP_BEGIN_HOP_CHECK:
        if (!need(1)) return false;
        line("if ((" + a + ") == 0.0f) {");
        ++indent;
        return true;
      case DGEN_HIP_UOP_BEGIN_LOOP: {
        if (!need(1)) return false;
        const int64_t step = u.imm[0] ? u.imm[0] : 1;
        if (step < 0) line("for (int i = (int)(" + a + ") - 1; i >= 0; i += " + std::to_string(step) + ") {");
        else line("for (unsigned i = 0; i < (unsigned)(" + a + "); i += " + std::to_string(step) + "u) {");
        ++indent;
        return true;
      }
      case DGEN_HIP_UOP_BEGIN_REVERSE_LOOP:
        if (!need(1)) return false;
        line("for (int i = (int)(" + a + ") - 1; i >= 0; i--) {");
        ++indent;
        return true;
      case DGEN_HIP_UOP_BEGIN_FOR_LOOP: {
        if (u.a.kind != DGEN_HIP_LAZY_VAR) return bad("block %d: beginForLoop needs a variable", index);
        if (!g(u.b, b)) return false;
        const std::string v = "t" + std::to_string(u.a.id);
        const std::string n = u.b.kind == DGEN_HIP_LAZY_CONST ? std::to_string((long long)u.b.value) + "u"
                                                                : "(unsigned)(" + b + ")";
        int_vars.insert(u.a.id);
        line("for (unsigned " + v + " = 0; " + v + " < " + n + "; " + v + "++) {");
        ++indent;
        return true;
      }
      case DGEN_HIP_UOP_BEGIN_PARALLEL_RANGE: {
        if (u.value.kind != DGEN_HIP_LAZY_VAR) return bad("block %d: beginParallelRange needs a variable", index);
        pr_vars.insert(u.value.id);
        const std::string v = "_pr" + std::to_string(u.value.id);
        line("for (unsigned " + v + " = 0; " + v + " < " + std::to_string(u.imm[0]) + "u; " + v + "++) {");
        ++indent;
        return true;
      }
      case DGEN_HIP_UOP_BEGIN_RANGE: {
        std::string s0, s1;
        if (!lazy(u.a, true, s0) || !lazy(u.b, true, s1)) return false;
        line("if (id >= (unsigned)(" + s0 + ") && id < (unsigned)(" + s1 + ")) {");
        ++indent;
        return true;
      }
      case DGEN_HIP_UOP_END_IF:
      case DGEN_HIP_UOP_END_LOOP:
      case DGEN_HIP_UOP_END_RANGE:
      case DGEN_HIP_UOP_END_PARALLEL_RANGE:
      case DGEN_HIP_UOP_END_HOP_CHECK:
        if (indent <= 1) return bad("block %d: unbalanced end (op %d)", index, u.op);
        --indent;
        line("}");
        return true;
      // ---- indices and run parameters
      case DGEN_HIP_UOP_FRAME_INDEX:
        return assign(u, frame_override ? "_frameIndex" : base_idx());
      case DGEN_HIP_UOP_THREAD_INDEX:
        return assign(u, (parallel || blk.dispatch == DGEN_HIP_DISPATCH_FIXED_WITH_FRAME_LOOP ||
                          blk.dispatch == DGEN_HIP_DISPATCH_SELF_MANAGED_THREADS)
                             ? "id"
                             : "i");
      case DGEN_HIP_UOP_FRAME_COUNT:
        if (u.value.kind == DGEN_HIP_LAZY_EMPTY) return true;  // the renderer's marker
        return assign(u, "frameCount");
      case DGEN_HIP_UOP_HOST_SAMPLE_RATE:
        return assign(u, "hostSampleRate");
      case DGEN_HIP_UOP_SET_FRAME_INDEX:
        if (!need(1)) return false;
        if (frame_override) line("_frameIndex = (unsigned)(" + a + ");");
        else line("unsigned _frameIndex = (unsigned)(" + a + ");");
        frame_override = true;
        return true;
      case DGEN_HIP_UOP_OUTPUT: {
        if (!need(1)) return false;
        const std::string idx = "(unsigned long long)" + std::to_string(u.imm[0]) + "u * frameCount + " + frame_idx();
        line("{ const float _o = " + a + "; outputs[DG_O(" + idx + ")] = isfinite(_o) ? _o : 0.0f; }");
        return true;
      }
      case DGEN_HIP_UOP_INPUT: {
        const std::string idx = "(unsigned long long)" + std::to_string(u.imm[0]) + "u * frameCount + " + frame_idx();
        return assign(u, "inputs[DG_I(" + idx + ")]");
      }
      // ---- threadgroup scratch (Metal threadgroup memory -> LDS)
      case DGEN_HIP_UOP_THREADGROUP_ARRAY_DECL:
        if (u.imm[1] <= 0 || u.imm[1] > 16384) return bad("block %d: scratch of %lld floats", index, (long long)u.imm[1]);
        line("__shared__ float scratch_" + std::to_string(u.imm[0]) + "[" + std::to_string(u.imm[1]) + "];");
        return true;
      case DGEN_HIP_UOP_THREADGROUP_READ: {
        if (!need(1)) return false;
        return assign(u, "scratch_" + std::to_string(u.imm[0]) + "[(unsigned)(" + a + ")]");
      }
      case DGEN_HIP_UOP_THREADGROUP_WRITE:
        if (!need(2)) return false;
        line("scratch_" + std::to_string(u.imm[0]) + "[(unsigned)(" + a + ")] = " + b + ";");
        return true;
      case DGEN_HIP_UOP_THREADGROUP_BARRIER:
        line("__syncthreads();");
        return true;
      // ---- no code (view ops, markers, globals resolved to tape slots)
      case DGEN_HIP_UOP_NOP:
      case DGEN_HIP_UOP_DEFINE_GLOBAL:
      case DGEN_HIP_UOP_LOAD_GLOBAL:
      case DGEN_HIP_UOP_SET_THREAD_COUNT_SCALE:
        return true;
      default:
        return bad("block %d: op %d is not lowered by the generic renderer", index, u.op);
    }
  }

  // MetalRenderer.prepareSchedule's wrapping for the block's dispatch mode,
  // then the ops, then the closing braces.
  bool render() {
    parallel = blk.frame_order == DGEN_HIP_FRAME_PARALLEL;
    const int n = blk.dispatch_n;
    bool frame_loop = false, has_frames = false;
    switch (blk.dispatch) {
      case DGEN_HIP_DISPATCH_PER_FRAME_SCALED:
      case DGEN_HIP_DISPATCH_PER_FRAME_SCALED_TG1:
        if (n < 1) return bad("block %d: perFrameScaled(%d)", index, n);
        scale = n > 1 ? n : 0;
        break;
      default:
        break;
    }
    out += "extern \"C\" __global__ void dgen_block_" + std::to_string(index) +
           "(float* memory, float* t, float* outputs, const float* inputs, unsigned frameCount, float hostSampleRate, "
           "unsigned long long memFloats, unsigned long long tapeFloats, unsigned long long outFloats, "
           "unsigned long long inFloats) {\n";
    line("const unsigned id = blockIdx.x * blockDim.x + threadIdx.x;");
    line("float _noise = 0.0f;");
    line("(void)_noise; (void)inputs; (void)outputs; (void)t; (void)hostSampleRate;");
    if (blk.temporality == DGEN_HIP_TEMPORAL_STATIC) line("const unsigned i = 0;  // static block: no frame loop");
    switch (blk.dispatch) {
      case DGEN_HIP_DISPATCH_SINGLE_THREADED:
        line("if (id < 1u) {");
        ++indent;
        line("for (unsigned i = 0; i < frameCount; i += 1u) {");
        ++indent;
        frame_loop = has_frames = true;
        break;
      case DGEN_HIP_DISPATCH_SELF_MANAGED:
        line("if (id < 1u) {");
        ++indent;
        break;
      case DGEN_HIP_DISPATCH_SELF_MANAGED_THREADS:
      case DGEN_HIP_DISPATCH_STATIC_THREADS:
        if (n < 1) return bad("block %d: thread count %d", index, n);
        line("if (id < " + std::to_string(n) + "u) {");
        ++indent;
        break;
      case DGEN_HIP_DISPATCH_FIXED_WITH_FRAME_LOOP:
        if (n < 1) return bad("block %d: fixedWithFrameLoop(%d)", index, n);
        line("if (id < " + std::to_string(n) + "u) {");
        ++indent;
        line("for (unsigned i = 0; i < frameCount; i += 1u) {");
        ++indent;
        frame_loop = has_frames = true;
        break;
      case DGEN_HIP_DISPATCH_PER_FRAME:
      case DGEN_HIP_DISPATCH_PER_FRAME_TG1:
        line("if (id < frameCount) {");
        ++indent;
        has_frames = true;
        break;
      case DGEN_HIP_DISPATCH_PER_FRAME_SCALED:
      case DGEN_HIP_DISPATCH_PER_FRAME_SCALED_TG1:
        if (!parallel) {
          // one thread loops over frameCount * n iterations
          line("if (id < 1u) {");
          ++indent;
          line("for (unsigned i = 0; i < frameCount * " + std::to_string(n) + "u; i += 1u) {");
          ++indent;
          frame_loop = true;
        } else {
          line("if (id < frameCount * " + std::to_string(n) + "u) {");
          ++indent;
        }
        has_frames = true;
        break;
      default:
        return bad("block %d: dispatch mode %d is not lowered by the generic renderer", index, blk.dispatch);
    }
    (void)frame_loop;
    const int base_indent = indent;
    if (has_frames && blk.temporality == DGEN_HIP_TEMPORAL_HOP) {
      std::string cnt;
      if (!g(blk.hop_counter, cnt)) return false;
      line("if ((" + cnt + ") == 0.0f) {");
      ++indent;
    }
    if (blk.n_ops && !blk.ops) return bad("block %d: null ops", index);
    for (uint32_t k = 0; k < blk.n_ops; ++k)
      if (!emit(blk.ops[k])) return false;
    if (indent != (has_frames && blk.temporality == DGEN_HIP_TEMPORAL_HOP ? base_indent + 1 : base_indent))
      return bad("block %d: unbalanced begin/end ops", index);
    while (indent > 1) {
      --indent;
      line("}");
    }
    out += "}\n\n";
    return true;
  }
};

const char* kPrelude =
    "// generated by libdgen_hip (uop_render.cpp) from DGen UOp blocks\n"
    "#define DG_M(x) ((unsigned long long)(x) < memFloats ? (unsigned long long)(x) : memFloats - 1ull)\n"
    "#define DG_T(x) ((unsigned long long)(x) < tapeFloats ? (unsigned long long)(x) : tapeFloats - 1ull)\n"
    "#define DG_O(x) ((unsigned long long)(x) < outFloats ? (unsigned long long)(x) : outFloats - 1ull)\n"
    "#define DG_I(x) ((unsigned long long)(x) < inFloats ? (unsigned long long)(x) : inFloats - 1ull)\n"
    "__device__ __forceinline__ float dg_sign(float v) { return v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f); }\n\n";

}  // namespace

// The largest cell a block addresses directly (load/store/delay1/noise and
// the base cell of indexed accesses), for the launch-time arena check; -1
// if none.
int64_t block_max_cell(const dgen_hip_block& b) {
  int64_t m = -1;
  for (uint32_t k = 0; k < b.n_ops; ++k) {
    switch (b.ops[k].op) {
      case DGEN_HIP_UOP_LOAD:
      case DGEN_HIP_UOP_STORE:
      case DGEN_HIP_UOP_DELAY1:
      case DGEN_HIP_UOP_NOISE:
      case DGEN_HIP_UOP_MEMORY_READ:
      case DGEN_HIP_UOP_MEMORY_WRITE:
      case DGEN_HIP_UOP_MEMORY_ACCUMULATE:
      case DGEN_HIP_UOP_SIMD_BROADCAST_LOAD:
        m = std::max<int64_t>(m, b.ops[k].imm[0]);
        break;
      default:
        break;
    }
  }
  return m;
}

int render_blocks(const dgen_hip_block* blocks, uint32_t n, std::string& source) {
  if (n && !blocks) return fail(DGEN_HIP_E_INVALID, "render: null blocks");
  // tape slots written by static blocks hold one value (index 0)
  // (MetalRenderer.compile, MetalRenderer.swift:61-69)
  std::set<int> static_slots;
  for (uint32_t i = 0; i < n; ++i) {
    if (blocks[i].temporality != DGEN_HIP_TEMPORAL_STATIC) continue;
    for (uint32_t k = 0; k < blocks[i].n_ops; ++k) {
      const dgen_hip_uop& u = blocks[i].ops[k];
      if (u.op == DGEN_HIP_UOP_DEFINE_GLOBAL && u.a.kind == DGEN_HIP_LAZY_GLOBAL) static_slots.insert(u.a.id);
    }
  }
  source = kPrelude;
  for (uint32_t i = 0; i < n; ++i) {
    const dgen_hip_block& b = blocks[i];
    if (b.temporality < DGEN_HIP_TEMPORAL_FRAME || b.temporality > DGEN_HIP_TEMPORAL_STATIC)
      return fail(DGEN_HIP_E_INVALID, "render: block %u temporality %d", i, b.temporality);
    for (uint32_t k = 0; k < b.n_ops; ++k) {
      const dgen_hip_uop& u = b.ops[k];
      const bool cell_op = u.op == DGEN_HIP_UOP_LOAD || u.op == DGEN_HIP_UOP_STORE || u.op == DGEN_HIP_UOP_DELAY1 ||
                           u.op == DGEN_HIP_UOP_NOISE;
      if (cell_op && u.imm[0] < 0) return fail(DGEN_HIP_E_INVALID, "render: block %u op %u cell %lld", i, k,
                                               (long long)u.imm[0]);
    }
    Renderer r(b, (int)i, static_slots);
    if (!r.render()) return fail(DGEN_HIP_E_INVALID, "render: %s", r.err.c_str());
    source += r.out;
  }
  return 0;
}

// Threads of a block's launch (DispatchMode.threadCount, Renderer.swift:
// 71-86; a sequential perFrameScaled block runs its loop on one thread, as
// prepareSchedule's range guard makes it) and its workgroup size
// (threadGroupSize: 1 for the single-thread and threadgroup-scratch modes).
static void block_grid(const BlockInfo& b, uint32_t frames, uint64_t* threads, uint32_t* group) {
  const uint64_t n = (uint64_t)std::max(1, b.n);
  switch (b.dispatch) {
    case DGEN_HIP_DISPATCH_SINGLE_THREADED:
    case DGEN_HIP_DISPATCH_SELF_MANAGED:
      *threads = 1;
      *group = 1;
      return;
    case DGEN_HIP_DISPATCH_PER_FRAME:
      *threads = frames;
      *group = 256;
      return;
    case DGEN_HIP_DISPATCH_PER_FRAME_TG1:
      *threads = frames;
      *group = 1;
      return;
    case DGEN_HIP_DISPATCH_PER_FRAME_SCALED:
    case DGEN_HIP_DISPATCH_PER_FRAME_SCALED_TG1:
      *threads = b.frame_order == DGEN_HIP_FRAME_PARALLEL ? (uint64_t)frames * n : 1;
      *group = (b.dispatch == DGEN_HIP_DISPATCH_PER_FRAME_SCALED_TG1 || *threads == 1) ? 1 : 256;
      return;
    default:  // fixedWithFrameLoop, staticThreads, selfManagedThreads
      *threads = n;
      *group = 256;
      return;
  }
}

int launch_uop_block(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=block [1]=tape cell or -1 [2]=tape slots [3]=outputs cell or -1 [4]=output channels
  //      [5]=inputs cell or -1 [6]=input channels [7]=frames the cells hold
  // farg: [0]=graph sample rate
  const int64_t bi = op.arg[0], tape = op.arg[1], slots = op.arg[2], outc = op.arg[3], nout = op.arg[4];
  const int64_t inc = op.arg[5], nin = op.arg[6], cap = op.arg[7];
  DGEN_REQUIRE(bi >= 0 && (size_t)bi < L.n_blocks && L.blocks,
               "uop_block: block %lld of %zu (dgen_hip_set_blocks before dgen_hip_configure)", (long long)bi,
               L.n_blocks);
  DGEN_REQUIRE(cap >= 1 && cap <= (1ll << 30), "uop_block: frame capacity %lld", (long long)cap);
  DGEN_REQUIRE(slots >= 0 && nout >= 0 && nin >= 0, "uop_block: negative slot or channel count");
  const BlockInfo& b = L.blocks[bi];
  if (b.max_cell >= 0) DGEN_CHECK_CELL(L, 0, (uint64_t)b.max_cell + 1, "uop_block.cells");
  if (tape >= 0) DGEN_CHECK_CELL(L, tape, (uint64_t)std::max<int64_t>(1, slots * cap), "uop_block.tape");
  if (outc >= 0) DGEN_CHECK_CELL(L, outc, (uint64_t)std::max<int64_t>(1, nout * cap), "uop_block.outputs");
  if (inc >= 0) DGEN_CHECK_CELL(L, inc, (uint64_t)std::max<int64_t>(1, nin * cap), "uop_block.inputs");
  if (L.dry) return 0;
  uint64_t threads = 0;
  uint32_t group = 1;
  block_grid(b, L.frames, &threads, &group);
  if (threads == 0) return 0;
  const uint64_t blocks = (threads + group - 1) / group;
  DGEN_REQUIRE(blocks <= 0x7fffffffull, "uop_block: %llu threads", (unsigned long long)threads);
  // unused buffers point at the arena with one float, so every clamped
  // index stays inside an allocation
  float* mem = L.arena;
  float* tp = tape >= 0 ? cell(L, tape) : L.arena;
  float* op_ = outc >= 0 ? cell(L, outc) : L.arena;
  const float* ip = inc >= 0 ? cell(L, inc) : L.arena;
  unsigned frames = L.frames;
  float sr = host_rate(L, op.farg[0]);
  unsigned long long memf = L.arena_floats, tapef = tape >= 0 ? (unsigned long long)std::max<int64_t>(1, slots * cap) : 1;
  unsigned long long outf = outc >= 0 ? (unsigned long long)std::max<int64_t>(1, nout * cap) : 1;
  unsigned long long inf = inc >= 0 ? (unsigned long long)std::max<int64_t>(1, nin * cap) : 1;
  void* args[] = {&mem, &tp, &op_, &ip, &frames, &sr, &memf, &tapef, &outf, &inf};
  DGEN_HIP_TRY(hipModuleLaunchKernel(b.fn, (unsigned)blocks, 1, 1, group, 1, 1, 0, L.stream, args, nullptr));
  return 0;
}

}  // namespace dgen
