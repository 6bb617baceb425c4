// Host-side helpers shared by the C-ABI entry points: status/last-error
// handling, argument checks and the drop-in HIP_CHECK behaviour.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nvf_ops.h"

namespace nvf {

// Records `msg` as the calling thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks hipGetLastError() after a launch; NVF_OK or NVF_ERR_LAUNCH.
int launch_status(const char* what);

// The reference's HIP_CHECK (include/nanovllm/common.hpp:14-23) for drop-in
// entry points: print and exit(1) on a nonzero status.
void dropin_check(int status, const char* what);

// The Q4_K nibble order the drop-ins read (hip_embedding_qk, hip_matmul_qk), set
// process-wide by nvf_set_dropin_q4k_layout.
int dropin_q4k_layout();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// True if the byte ranges [a, a + an) and [b, b + bn) share a byte.
inline bool bytes_overlap(const void* a, int64_t an, const void* b, int64_t bn) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return an > 0 && bn > 0 && pa < pb + (uintptr_t)bn && pb < pa + (uintptr_t)an;
}

inline int dtype_bytes(int dt) { return dt == NVF_F32 ? 4 : 2; }
inline bool dtype_ok(int dt) { return dt == NVF_F32 || dt == NVF_F16 || dt == NVF_BF16; }

}  // namespace nvf

// Expands `BODY` with `T` bound to the storage type of `dt`.
#define NVF_DISPATCH_DTYPE(dt, T, BODY)      \
  do {                                       \
    if ((dt) == NVF_F32) {                   \
      using T = float;                       \
      BODY;                                  \
    } else if ((dt) == NVF_F16) {            \
      using T = _Float16;                    \
      BODY;                                  \
    } else {                                 \
      using T = __bf16;                      \
      BODY;                                  \
    }                                        \
  } while (0)
