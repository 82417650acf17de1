// Status of a host-side call: the facade's Result<_, Error(String)> (nuvec.rs:18-38). A failed
// call returns its MRUN_ERR_* code and leaves the message for mrun_last_error() (per thread).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "mrun_moe.h"

namespace mrun {

struct Status {
    int code = MRUN_OK;
    std::string msg;
    bool ok() const { return code == MRUN_OK; }
};

inline Status Ok() { return Status{}; }
inline Status Err(int code, std::string msg) { return Status{code, std::move(msg)}; }

// Records the status as the thread's last error (cleared on success); returns its code.
int report(const Status &s);

inline Status hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return Ok();
    return Err(MRUN_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace mrun

#define TRY(expr)                         \
    do {                                  \
        ::mrun::Status _s = (expr);       \
        if (!_s.ok()) return _s;          \
    } while (0)
#define TRY_HIP(expr, what) TRY(::mrun::hip_status((expr), (what)))
