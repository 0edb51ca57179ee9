// Error reporting shared by the C-ABI entry points: every entry point returns
// a hipError_t as int; a failed argument check also records a message that
// ek_last_error() returns (per host thread).
#pragma once

#include <hip/hip_runtime.h>
#include <cstring>

hipError_t ek_fail(hipError_t code, const char* msg);
void ek_clear_error();

#define EK_GUARD() ek_clear_error()
