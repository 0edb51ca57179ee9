// Error reporting shared by the C-ABI entry points: every entry point returns
// a hipError_t as int; a failed argument check also records a message that
// ek_last_error() returns (per host thread).
#pragma once

#include <hip/hip_runtime.h>
#include <cstring>

hipError_t ek_fail(hipError_t code, const char* msg);
void ek_clear_error();

#define EK_GUARD() ek_clear_error()

// Polls a bounded device-side wait may spend before it gives up: `dflt`
// unless ek_set_wait_limit() chose another bound (read at launch time, so a
// captured graph keeps the bound it was captured with).
int64_t ek_wait_limit(int64_t dflt);
