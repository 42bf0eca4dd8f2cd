// Helpers shared by the C ABI translation units (capi.cpp: mat-vec and attention; decode.cpp: the decode-step
// glue and driver). Not part of the public interface.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/p1x.h"
#include "launch.h"

namespace p1x::capi {

extern thread_local std::string g_error;
int fail(int code, const std::string& why);  // records the reason for p1x_last_error, returns code
int hip_fail(hipError_t e, const char* what);
int ensure_init();

int block_elems(int wtype);  // 0 bytes for an unknown type
int block_bytes(int wtype);
size_t align256(size_t n);
size_t q8_1_bytes(int64_t K, int64_t ncols);
bool aligned(const void* p, size_t n);
int check_matvec(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, int64_t ncols, const float* y,
                 int max_cols);

// Attention argument checks and kernel arguments shared by the attention entry points and the decode driver.
size_t fa_workspace(const p1x_attn_params* p);
int fa_prepare(const p1x_attn_params* p, const float* q, const uint16_t* k, const uint16_t* v,
               const p1x_kv_strides* strides, const float* mask, const int32_t* kv_len, float* o, float* lse, void* ws,
               size_t ws_bytes, FaArgs& a, bool kv_f16 = true);

}  // namespace p1x::capi
