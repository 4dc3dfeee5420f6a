// common.h - shared helpers of libjepa (logging, HIP error checks, small types).
#pragma once
#include <cstdint>
#include <cstddef>
#include <string>
#include <mutex>

#ifndef JEPA_VERSION
#define JEPA_VERSION "0.5.0-mi355x"
#endif

// Diagnostics: every line goes to stderr and to a thread-local capture buffer (jepa_error_text),
// the reference's contract (include/jepa.h:596-610, src/jepa.cpp:16-36).
void jepa_log(const char * fmt, ...) __attribute__((format(printf, 1, 2)));

// Serialises the library's device allocations and frees, model uploads and hipGraph captures across
// threads. A stream capture fails when another thread allocates, frees or copies through the null
// stream while it is open; contexts in different threads share one device, so every such call of
// the library holds this lock. Kernel launches, graph replays and copies on a context's own
// non-blocking stream do not need it.
std::recursive_mutex & jepa_hip_mutex();

// ggml_type ids as stored in GGUF tensor infos
enum ggml_type_id : int {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q8_1 = 9,
    T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15, T_BF16 = 30,
};

// block size / bytes per block of a ggml type; {0, 0} for types this library does not know
struct type_traits { int64_t blck; int64_t bytes; const char * name; };
type_traits ggml_traits(int type);
