// CPU check of the exact parallel fold's arithmetic (nd_fold.h): a host
// model of the device algorithm -- terms split into per-thread chunks, an
// fp32 prefix built as the device builds it (chunk prefix, 64-lane
// Hillis-Steele scan, waves in order), binade bounds, run maps, and the
// folded sequence -- against the plain sequential loop, over adversarial
// inputs.  Prints one line per generator: cases, mismatches, mean items.
#include "nd_fold.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

uint64_t g_state = 0x9e3779b97f4a7c15ull;
uint64_t next_u64()
{
    uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
double unif() { return double(next_u64() >> 11) * 0x1p-53; }
double gauss()
{
    const double u1 = unif() + 1e-300, u2 = unif();
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

float serial_fold(const float *a, int n)
{
    float s = 0.0f;
    for (int i = 0; i < n; ++i) s += a[i];
    return s;
}

// The device algorithm, modelled on the host.  Returns the fold and the
// number of items of the folded sequence (-1 when the plain loop ran).
float model_fold(const float *a, int n, int nt, int *items_out)
{
    *items_out = -1;
    if (n == 0) return 0.0f;
    const int c = (n + nt - 1) / nt;
    if (c > 16) return serial_fold(a, n);
    bool bad = false;
    std::vector<float> loc(n), tot(nt, 0.0f);
    for (int t = 0; t < nt; ++t) {
        float p = 0.0f;
        for (int j = 0; j < c && t * c + j < n; ++j) {
            const float x = a[t * c + j];
            bad |= nd_f2u(x) >= 0x7f800000u;
            p += x;
            loc[t * c + j] = p;
        }
        tot[t] = p;
        bad |= !(p < 0x1p110f);
    }
    if (bad) return serial_fold(a, n);
    // exclusive prefix of the chunk totals: Hillis-Steele inside each
    // 64-lane wave, the previous lane's inclusive value, plus the waves
    // before in order
    std::vector<float> excl(nt);
    float wave_base = 0.0f;
    for (int w0 = 0; w0 < nt; w0 += 64) {
        float x[64];
        for (int l = 0; l < 64; ++l) x[l] = tot[w0 + l];
        for (int off = 1; off < 64; off <<= 1) {
            float y[64];
            for (int l = 0; l < 64; ++l) y[l] = l >= off ? x[l] + x[l - off] : x[l];
            std::memcpy(x, y, sizeof(x));
        }
        for (int l = 0; l < 64; ++l) excl[w0 + l] = wave_base + (l ? x[l - 1] : 0.0f);
        wave_base += x[63];
    }
    const float dl = nd_fold_delta(n, c), cm = 1.0f - dl, cp = 1.0f + dl;
    // items of the folded sequence, in order: crossing terms and ties as
    // they are, each run of in-binade steps as its units' sum times u
    std::vector<float> items;
    bool open = false;
    int openG = 0;
    float D = 0.0f;
    auto flush = [&]() {
        if (!open) return;
        items.push_back(nd_fold_scale(D, openG));
        open = false;
    };
    for (int t = 0; t < nt; ++t) {
        const int i0 = t * c;
        if (i0 >= n) break;
        const int len = n - i0 < c ? n - i0 : c;
        int before = nd_fold_point_cls(excl[t], cm, cp);
        for (int j = 0; j < len; ++j) {
            const int after = nd_fold_point_cls(excl[t] + loc[i0 + j], cm, cp);
            float r;
            const bool in = nd_fold_units(a[i0 + j], before, r) && before && before == after;
            if (in) {
                if (open && openG != before) {  // cannot happen with sound bounds
                    std::fprintf(stderr, "class change inside a run at %d\n", i0 + j);
                    std::exit(2);
                }
                D = open ? D + r : r;
                open = true;
                openG = before;
            } else {
                flush();
                items.push_back(a[i0 + j]);
            }
            before = after;
        }
    }
    flush();
    float s = 0.0f;
    for (float it : items) s += it;
    *items_out = int(items.size());
    return s;
}

float pick_scale()
{
    static const float sc[] = {1.0f, 1e-3f, 1e3f, 1e-20f, 1e20f, 0x1p-140f, 0x1p-126f, 1e-38f};
    return sc[next_u64() % (sizeof(sc) / sizeof(sc[0]))];
}

// generators
void gen(int kind, std::vector<float> &v)
{
    const int n = int(v.size());
    const float scale = pick_scale();
    switch (kind) {
    case 0:  // squares of normals (norms)
        for (auto &x : v) {
            const float g = float(gauss()) * scale;
            x = g * g;
        }
        break;
    case 1:  // exps of scores (softmax sums)
        for (auto &x : v) x = std::exp(float(gauss() * 3.0) - 6.0f);
        break;
    case 2:  // few significant bits: frequent exact ties
        for (auto &x : v) {
            const int m = 1 + int(next_u64() % 15);
            const int e = int(next_u64() % 40) - 20;
            x = std::ldexp(float(m), e);
        }
        break;
    case 3:  // zeros mixed in, long zero prefix
        for (int i = 0; i < n; ++i) {
            const bool zero = i < n / 3 || next_u64() % 4 == 0;
            const float g = float(gauss());
            v[i] = zero ? 0.0f : g * g * scale;
        }
        break;
    case 4:  // subnormals and tiny normals
        for (auto &x : v) x = nd_u2f(uint32_t(next_u64() % 0x01800000u));
        break;
    case 5:  // powers of two only
        for (auto &x : v) x = std::ldexp(1.0f, int(next_u64() % 24) - 12);
        break;
    case 6:  // each term about the running sum: a crossing every step
        {
            double s = 1e-3;
            for (auto &x : v) {
                x = float(s * (0.5 + unif()));
                s += x;
                if (s > 1e30) s = 1e-3;
            }
        }
        break;
    case 7:  // one large term early, then small ones that vanish or round
        for (int i = 0; i < n; ++i) {
            const float g = float(gauss());
            v[i] = i == n / 7 ? 1e8f : g * g;
        }
        break;
    case 8:  // random bit patterns of non-negative finite floats
        for (auto &x : v) {
            uint32_t u;
            do u = uint32_t(next_u64()) & 0x7fffffffu; while (u >= 0x6f000000u);
            x = nd_u2f(u);
        }
        break;
    case 9:  // uniform [0, 1) with 24-bit mantissas hitting half-ulps
        for (auto &x : v) x = float(next_u64() >> 40) * 0x1p-24f;
        break;
    default:  // values from a tiny set, in a block of equal terms
        {
            const float base = float(1 + next_u64() % 7) * 0.125f * scale;
            for (auto &x : v) x = next_u64() % 8 ? base : base * 3.0f;
        }
        break;
    }
}

}  // namespace

int main(int argc, char **argv)
{
    const int cases = argc > 1 ? std::atoi(argv[1]) : 2000;
    if (argc > 2) g_state = std::strtoull(argv[2], nullptr, 0);
    static const int sizes[] = {1, 2, 3, 7, 64, 65, 255, 256, 257, 768, 1000, 1024, 2048, 3072, 4095};
    static const int threads[] = {256, 1024};
    int failures = 0;
    for (int kind = 0; kind <= 10; ++kind) {
        long long items = 0, runs = 0, bad = 0, fallback = 0;
        for (int k = 0; k < cases; ++k) {
            const int n = sizes[next_u64() % (sizeof(sizes) / sizeof(sizes[0]))];
            const int nt = threads[next_u64() % 2];
            std::vector<float> v(n);
            gen(kind, v);
            int it;
            const float got = model_fold(v.data(), n, nt, &it);
            const float want = serial_fold(v.data(), n);
            if (nd_f2u(got) != nd_f2u(want)) {
                if (bad < 5)
                    std::printf("MISMATCH kind %d n %d nt %d: got %a want %a\n", kind, n, nt, got, want);
                ++bad;
            }
            if (it < 0) {
                ++fallback;
            } else {
                items += it;
                ++runs;
            }
        }
        std::printf("kind %2d cases %d mismatches %lld fallback %lld mean_items %.1f\n", kind, cases, bad,
                    fallback, runs ? double(items) / runs : 0.0);
        failures += int(bad);
    }
    std::printf("%s\n", failures ? "FAIL" : "OK");
    return failures ? 1 : 0;
}
