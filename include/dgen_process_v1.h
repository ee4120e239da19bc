/*
 * dgen_process_v1.h -- the reference's process-function ABI, exported by
 * libdgen_hip.so so that a host that drives DGen process-function libraries
 * (dlopen, dlsym "dgen_process_v1", a zeroed state block per instance) can
 * drive a schedule of this backend unchanged.
 *
 * Names, types and signatures are the reference's
 * (toolchain/include/dgen_runtime.h:252-291; Swift view Types.swift:5-26).
 * A host that already includes the reference's dgen_runtime.h uses its
 * declarations instead of this header: the layouts are the same.
 *
 * Which schedule the exports run is chosen with dgen_hip_process_bind
 * (dgen_hip.h): a configured context with process ports, and the range of
 * its arena that is the graph's `memory` -- the cells the reference keeps in
 * the host's state block (parameters, tensors and the state cells carried
 * between calls).  The host sizes the block with
 * dgen_hip_process_memory_size() (at least 1024 floats, as the reference's
 * runtime does, Runtime.swift:228-237), zeroes it and writes its parameters
 * into it at their cell offsets (injectTensorData, Tensor.swift:320-330).
 */
#ifndef DGEN_PROCESS_V1_H
#define DGEN_PROCESS_V1_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DGEN_ABI_VERSION_V1 1u

typedef struct DGenProcessContextV1 {
  uint32_t abi_version; /* DGEN_ABI_VERSION_V1 */
  uint32_t struct_size; /* sizeof(DGenProcessContextV1) */
  float sample_rate;    /* host sample rate of this call; 0: the graph's own */
  uint32_t reserved;
} DGenProcessContextV1;

/* The reference's host FFT services (vDSP-backed on its C backend).  This
 * backend computes every transform on the GPU and never reads them, so the
 * type is only named here. */
typedef struct DGenHostServicesV1 DGenHostServicesV1;

/* One block of the bound schedule (dgen_runtime.h:283-289):
 *   inputs[c][i] / outputs[c][i]: channel c, frame i, for the bound
 *     context's process ports (dgen_hip_set_process_ports), frame_count in
 *     [1, the context's max_frames];
 *   state: the caller's block of dgen_hip_process_memory_size() floats.  Its
 *     [0, memory_floats) is the graph's memory: it is copied to the bound
 *     arena range before the block runs and copied back after it, so the
 *     carried state lives in the block (a host that zeroes it resets the
 *     graph, and each block is an independent instance of the graph);
 *   context: its sample_rate is the host rate of the block when abi_version
 *     is DGEN_ABI_VERSION_V1 and struct_size covers the struct (the
 *     reference's test, CRenderer.swift:357-359); otherwise, or when NULL,
 *     the graph's own rate;
 *   host: not read.
 * Synchronous.  Returns nothing, as the reference's does: on a failure (bad
 * arguments, a frame count the schedule cannot run, a device error) the
 * bound schedule's output channels are set to 0 for frame_count frames and
 * the state block is left as it was; with nothing bound the call changes
 * nothing.  Either way dgen_hip_last_error() on the calling thread holds the
 * message.  Calls are serialised internally. */
void dgen_process_v1(const float* const* inputs, float* const* outputs, uint32_t frame_count, void* state,
                     const DGenProcessContextV1* context, const DGenHostServicesV1* host);

/* The reference C backend's parameter entry point, a no-op there
 * (CRenderer.swift:341-347): parameters live in the state block, which the
 * host writes directly.  A no-op here too. */
void dgen_set_param_value_v1(int32_t cell_id, float value);

#ifdef __cplusplus
}
#endif

#endif /* DGEN_PROCESS_V1_H */
