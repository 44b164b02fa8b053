// Host check of the one-thread-at-a-time claim (needle-rs_amd/csrc/nd_owner.h)
// that guards contexts and batches: re-entry on the owning thread, refusal
// on another thread while held, release, and no lost claim when threads race.
#include <cstdio>
#include <thread>
#include <vector>

#include "nd_owner.h"

static int failures = 0;
#define CHECK(c)                                              \
    do {                                                      \
        if (!(c)) {                                           \
            std::printf("FAIL line %d: %s\n", __LINE__, #c);  \
            ++failures;                                       \
        }                                                     \
    } while (0)

static bool claim_on_other_thread(nd::Owner &o)
{
    bool ok = false;
    std::thread t([&] {
        ok = nd::owner_claim(o);
        if (ok) nd::owner_release(o);
    });
    t.join();
    return ok;
}

int main()
{
    nd::Owner o;
    CHECK(claim_on_other_thread(o));        // free: another thread may claim
    CHECK(nd::owner_claim(o));              // this thread claims
    CHECK(nd::owner_claim(o));              // and re-enters
    CHECK(!claim_on_other_thread(o));       // held: refused elsewhere
    nd::owner_release(o);
    CHECK(!claim_on_other_thread(o));       // still held once
    nd::owner_release(o);
    CHECK(claim_on_other_thread(o));        // free again
    CHECK(o.depth == 0);

    // Threads racing for one object: while a claim is held nobody else gets
    // it, so the counter below is never touched by two threads at once.
    nd::Owner r;
    long inside = 0, max_inside = 0, done = 0;
    std::vector<std::thread> ts;
    for (int i = 0; i < 8; ++i)
        ts.emplace_back([&] {
            for (int k = 0; k < 20000; ++k) {
                if (!nd::owner_claim(r)) continue;
                const long n = ++inside;
                if (n > max_inside) max_inside = n;
                ++done;
                --inside;
                nd::owner_release(r);
            }
        });
    for (auto &t : ts) t.join();
    CHECK(max_inside == 1);
    CHECK(done > 0);
    CHECK(r.depth == 0);
    std::printf(failures ? "FAILED\n" : "OK\n");
    return failures ? 1 : 0;
}
