// Internal (non-ABI) declarations shared by the gdnx translation units.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/gdnx.h"

namespace gdnx {

struct DeltaArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* ae;
  const float* aw;
  const float* g;
  const float* s0;
  void* y;
  float* s_out;
  void* chunk_states;
  int B, T, H, M, D, C, dtype;
};

struct DeltaBwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* ae;
  const float* aw;
  const float* g;
  const void* dy;
  const float* ds_final;
  const void* s_stash;
  void* ds_stash;
  void* dq;
  void* dk;
  void* dv;
  float* dae;
  float* daw;
  float* dg;
  float* ds0;
  int B, T, H, M, D, C, dtype;
};

// Record an error message for gdnx_last_error(); returns code.
int set_error(int code, const char* fmt, ...);
// Check hipGetLastError() after a launch.
int check_launch(const char* what);

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* ae;
  const float* aw;
  const float* g;
  float* state;
  void* y;
  int NS, H, M, D, dtype;
};

int decode_dispatch(const DecodeArgs& a, hipStream_t stream);
int delta_fwd_dispatch(const DeltaArgs& a, hipStream_t stream);
int delta_bwd_dispatch(const DeltaBwdArgs& a, int stages, hipStream_t stream);
int delta_chunk_size(int D, int dtype);
int delta_train_chunk_size(int D, int dtype);

}  // namespace gdnx
