// One host thread at a time inside calls on an object (a context, a batch):
// the owner's thread id, claimed on entry and released on exit.  Host-only
// and free of HIP, so the CPU tests build it with the host compiler.
#pragma once

#include <atomic>
#include <thread>

namespace nd {

struct Owner {
    std::atomic<std::thread::id> id{};
    int depth = 0;  // touched by the owning thread only
};

// Claims `o` for the calling thread: false if another thread holds it.  The
// owning thread may claim again (an entry point that calls another on the
// same object); each claim is undone by one owner_release.
inline bool owner_claim(Owner &o)
{
    const std::thread::id me = std::this_thread::get_id();
    std::thread::id cur{};
    if (!o.id.compare_exchange_strong(cur, me, std::memory_order_acquire) && cur != me)
        return false;
    ++o.depth;
    return true;
}

inline void owner_release(Owner &o)
{
    if (--o.depth == 0) o.id.store(std::thread::id{}, std::memory_order_release);
}

}  // namespace nd
