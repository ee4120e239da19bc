/* A process-function host in C, as the reference's runtime drives a DGen
 * process library (Sources/DGen/Runtime.swift:728-787): dlopen the library,
 * dlsym dgen_process_v1 / dgen_set_param_value_v1 by name, allocate and zero
 * a state block, and call one block.  Built and run by tests/test_abi.py on a
 * host without a GPU, where nothing is bound: the block must return with
 * its outputs silenced and a message, not abort. */
#include <dlfcn.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dgen_process_v1.h"

typedef void (*process_fn)(const float* const*, float* const*, uint32_t, void*, const DGenProcessContextV1*,
                           const DGenHostServicesV1*);
typedef void (*param_fn)(int32_t, float);
typedef uint64_t (*size_fn)(void);
typedef const char* (*err_fn)(void);

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  void* h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
  if (!h) {
    fprintf(stderr, "dlopen: %s\n", dlerror());
    return 3;
  }
  process_fn process = (process_fn)dlsym(h, "dgen_process_v1");
  param_fn set_param = (param_fn)dlsym(h, "dgen_set_param_value_v1");
  size_fn mem_size = (size_fn)dlsym(h, "dgen_hip_process_memory_size");
  err_fn last_error = (err_fn)dlsym(h, "dgen_hip_last_error");
  if (!process || !set_param || !mem_size || !last_error) return 4;
  if (mem_size() != 0) return 5; /* nothing bound yet */
  float* state = (float*)calloc(1024, sizeof(float));
  float out0[64];
  for (int i = 0; i < 64; ++i) out0[i] = 1.0f;
  float* outs[1] = {out0};
  DGenProcessContextV1 ctx = {DGEN_ABI_VERSION_V1, (uint32_t)sizeof(DGenProcessContextV1), 44100.0f, 0u};
  set_param(0, 0.5f);
  process(NULL, outs, 64, state, &ctx, NULL);
  printf("%s\n", last_error());
  const int ok = strstr(last_error(), "no schedule bound") != NULL && state[0] == 0.0f;
  free(state);
  return ok ? 0 : 6;
}
