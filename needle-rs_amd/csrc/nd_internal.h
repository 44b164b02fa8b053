// Internal plumbing shared by the HIP translation units: the context, the
// per-thread error message and launch-checking helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <string>

#include "needle_amd.h"
#include "nd_owner.h"

struct nd_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool owns_stream = false;
    int num_cus = 0;
    // Growable device workspace for split-K partials.  Owned by the context,
    // reused by every call on it; calls on one context are stream-ordered,
    // and only one host thread is inside a call on it at a time (`owner`).
    void *work = nullptr;
    size_t work_bytes = 0;
    nd::Owner owner;
};

namespace nd {

// Records a printf-style message for nd_last_error() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Maps a failed HIP call to ND_ERR_HIP with the call's text.
int hip_fail(hipError_t e, const char *what);

// owner_claim with an error: ND_ERR_BUSY if another thread is inside a call
// on the object (`what` names it in the message); release() undoes one claim.
int claim(Owner &o, const char *what);
inline void release(Owner &o) { owner_release(o); }

// The scope of one entry-point call on a context: claims the context for
// the calling thread and makes its device current; `rc` is ND_OK or the
// error.  The claim ends with the scope.
class Entry {
public:
    explicit Entry(nd_ctx *ctx);
    ~Entry();
    Entry(const Entry &) = delete;
    Entry &operator=(const Entry &) = delete;
    int rc = ND_OK;

private:
    nd_ctx *ctx_ = nullptr;
};

// The same for an object other than a context (a batch).
class Hold {
public:
    Hold(Owner &o, const char *what) : o_(o), rc(claim(o, what)) {}
    ~Hold()
    {
        if (rc == ND_OK) release(o_);
    }
    Hold(const Hold &) = delete;
    Hold &operator=(const Hold &) = delete;

private:
    Owner &o_;

public:
    int rc;
};

// Ensures the context workspace holds at least `bytes`.
int workspace(nd_ctx *ctx, size_t bytes, void **out);

// Looks up, once per device and with that device current, the device
// address of the no-allocation entry point's scratch array.
int noalloc_setup(int device);

// Checks the launch that was just enqueued.
int check_launch(const char *kernel);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace nd

#define ND_HIP(call)                                        \
    do {                                                    \
        hipError_t e_ = (call);                             \
        if (e_ != hipSuccess) return nd::hip_fail(e_, #call); \
    } while (0)

// First statement of an entry point that takes a context.
#define ND_ENTER(ctx)              \
    nd::Entry nd_entry_(ctx);      \
    if (nd_entry_.rc) return nd_entry_.rc

#define ND_REQUIRE(cond, ...)                                  \
    do {                                                       \
        if (!(cond)) return nd::fail(ND_ERR_ARG, __VA_ARGS__); \
    } while (0)
