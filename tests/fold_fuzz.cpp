// CPU check of the exact parallel fold's arithmetic (nd_fold.h), two ways,
// both against the plain sequential loop over adversarial inputs:
//  - model_fold: the algorithm as a sequence -- terms split into
//    per-thread chunks, an fp32 prefix (chunk prefix, a 64-lane
//    Hillis-Steele scan, waves in order), binade bounds, run maps and the
//    folded sequence;
//  - emulate_device: nd_fold_nonneg lane for lane -- its 64-lane DPP scans
//    (row shifts, row broadcasts under their row masks, wave shifts, the
//    value 0 where a lane has no source), the carry scan of nd_fold_then,
//    the tail, lead and count rules, and every thread writing its items at
//    obase + lead + cex.  Each item must be written once, and the items
//    must equal, in count and order, the sequential list built for the same
//    prefix.
// Prints one line per generator (cases, mismatches, mean items), then how
// many cases the emulation covered and how many runs it saw cross a wave
// edge.
#include "nd_fold.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

constexpr int kNdFoldItemsHost = 512;  // nd_fold.h's kNdFoldItems

uint64_t g_state = 0x9e3779b97f4a7c15ull;
int g_nt = 256;          // threads of the case being generated
long long g_leads = 0;   // runs written by the next wave's lane 0
long long g_inner_tails = 0;  // runs written before the next chunk's crossing term
uint64_t g_edge_kind = 0;
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

// ---- the device code of nd_fold_nonneg, lane for lane -------------------------
// NT threads in NW = NT / 64 waves.  The DPP moves are modelled with their
// row and wave semantics: a lane with no source (or in a row the row mask
// leaves out) gets the old value, 0.
// nd_fold.h's NdFoldCarry (device-only there): flags bit 0 the span has a
// crossing term, bit 1 a run is open at its end, bits 2+ the run's binade;
// D the run's sum of units.
struct NdFoldCarry {
    int flags;
    float D;
};

enum Dpp { ROW_SHR1, ROW_SHR2, ROW_SHR4, ROW_SHR8, ROW_BCAST15, ROW_BCAST31, WAVE_SHR1, WAVE_SHL1 };

template <typename T>
void dpp64(const T *src, T *dst, Dpp op, T zero)
{
    for (int l = 0; l < 64; ++l) {
        const int row = l >> 4, rl = l & 15;
        int from = -1;
        switch (op) {
        case ROW_SHR1: from = rl >= 1 ? l - 1 : -1; break;
        case ROW_SHR2: from = rl >= 2 ? l - 2 : -1; break;
        case ROW_SHR4: from = rl >= 4 ? l - 4 : -1; break;
        case ROW_SHR8: from = rl >= 8 ? l - 8 : -1; break;
        case ROW_BCAST15: from = (row == 1 || row == 3) ? row * 16 - 1 : -1; break;  // row mask 0xa
        case ROW_BCAST31: from = (row == 2 || row == 3) ? 31 : -1; break;          // row mask 0xc
        case WAVE_SHR1: from = l >= 1 ? l - 1 : -1; break;
        case WAVE_SHL1: from = l <= 62 ? l + 1 : -1; break;
        }
        dst[l] = from >= 0 ? src[from] : zero;
    }
}

NdFoldCarry then_h(NdFoldCarry a, NdFoldCarry b)  // nd_fold_then
{
    const bool bkind = b.flags & 1, bex = (b.flags >> 1) & 1, aex = (a.flags >> 1) & 1;
    NdFoldCarry r;
    r.flags = bkind ? b.flags : (bex ? ((a.flags & 1) | 2 | (b.flags & ~3)) : a.flags);
    r.D = bkind ? b.D : (bex ? (aex ? a.D + b.D : b.D) : a.D);
    return r;
}

void scan_add64(float *v)  // nd_fold_scan_add
{
    static const Dpp ops[6] = {ROW_SHR1, ROW_SHR2, ROW_SHR4, ROW_SHR8, ROW_BCAST15, ROW_BCAST31};
    for (Dpp op : ops) {
        float t[64];
        dpp64(v, t, op, 0.0f);
        for (int l = 0; l < 64; ++l) v[l] = v[l] + t[l];
    }
}

void scan_int64(int *v)  // nd_fold_scan_int
{
    static const Dpp ops[6] = {ROW_SHR1, ROW_SHR2, ROW_SHR4, ROW_SHR8, ROW_BCAST15, ROW_BCAST31};
    for (Dpp op : ops) {
        int t[64];
        dpp64(v, t, op, 0);
        for (int l = 0; l < 64; ++l) v[l] = v[l] + t[l];
    }
}

void scan_carry64(NdFoldCarry *f)  // nd_fold_scan_carry
{
    static const Dpp ops[6] = {ROW_SHR1, ROW_SHR2, ROW_SHR4, ROW_SHR8, ROW_BCAST15, ROW_BCAST31};
    for (Dpp op : ops) {
        NdFoldCarry t[64];
        dpp64(f, t, op, NdFoldCarry{0, 0.0f});
        for (int l = 0; l < 64; ++l) f[l] = then_h(t[l], f[l]);
    }
}

// What the device computes: the fold (thread 0's result), and through the
// out-parameters the chunks' exclusive prefixes and the items array as the
// threads write it (-1 items: the plain loop ran).
float emulate_device(const float *v, int n, int NT, int CMAX, std::vector<float> &excl_out,
                     std::vector<float> &items_out, int *total_out)
{
    const int NW = NT / 64;
    *total_out = -1;
    const int c = (n + NT - 1) / NT;
    if (n < 128 || c > CMAX) return serial_fold(v, n);
    std::vector<float> x(size_t(NT) * CMAX), loc(size_t(NT) * CMAX);
    std::vector<int> len(NT);
    std::vector<float> p(NT);
    bool bad = false;
    for (int t = 0; t < NT; ++t) {
        const int i0 = t * c;
        len[t] = n - i0 < 0 ? 0 : (n - i0 < c ? n - i0 : c);
        float acc = 0.0f;
        for (int j = 0; j < CMAX; ++j) {
            const int i = i0 + j < n ? i0 + j : n - 1;
            const float xv = j < len[t] ? v[i] : 0.0f;
            x[size_t(t) * CMAX + j] = xv;
            bad |= nd_f2u(xv) >= 0x7f800000u;
            acc += xv;
            loc[size_t(t) * CMAX + j] = acc;
        }
        p[t] = acc;
        bad |= !(acc < 0x1p110f);
    }
    if (bad) return serial_fold(v, n);
    // 1. the fp32 exclusive prefix of the chunk totals
    std::vector<float> excl(NT), wtot(NW);
    for (int w = 0; w < NW; ++w) {
        float incl[64], lex[64];
        for (int l = 0; l < 64; ++l) incl[l] = p[w * 64 + l];
        scan_add64(incl);
        dpp64(incl, lex, WAVE_SHR1, 0.0f);
        wtot[w] = incl[63];
        for (int l = 0; l < 64; ++l) excl[w * 64 + l] = lex[l];
    }
    for (int t = 0; t < NT; ++t) {
        const int w = t >> 6;
        float base = 0.0f;
        if (NW > 1)
            for (int k = 0; k < NW - 1; ++k) base += k < w ? wtot[k] : 0.0f;
        excl[t] = base + excl[t];
    }
    excl_out = excl;
    // 2. binades, in-binade steps and units, runs and item counts per chunk
    const float dl = nd_fold_delta(n, c), cm = 1.0f - dl, cp = 1.0f + dl;
    std::vector<uint32_t> inm(NT);
    std::vector<float> rr(size_t(NT) * CMAX), runD(NT);
    std::vector<int> gg(size_t(NT) * CMAX), runG(NT), count(NT), first_bound(NT), any_bound(NT), open(NT);
    for (int t = 0; t < NT; ++t) {
        int before = nd_fold_point_cls(excl[t], cm, cp);
        float D = 0.0f;
        int G = 0, cnt = 0;
        bool op = false, anyb = false, fb = false;
        uint32_t m = 0;
        for (int j = 0; j < CMAX; ++j) {
            const bool valid = j < len[t];
            const int after = nd_fold_point_cls(excl[t] + loc[size_t(t) * CMAX + j], cm, cp);
            float r;
            const bool ok = nd_fold_units(x[size_t(t) * CMAX + j], before, r);
            const bool in = valid && ok && before != 0 && before == after;
            const bool bound = valid && !in;
            rr[size_t(t) * CMAX + j] = r;
            gg[size_t(t) * CMAX + j] = before;
            m |= in ? 1u << j : 0u;
            D = in ? (op ? D + r : r) : D;
            G = in ? before : G;
            if (j == 0) fb = bound;
            cnt += bound ? (op ? 2 : 1) : 0;
            anyb |= bound;
            op = in ? true : (bound ? false : op);
            before = valid ? after : before;
        }
        inm[t] = m;
        runD[t] = D;
        runG[t] = G;
        count[t] = cnt;
        first_bound[t] = fb;
        any_bound[t] = anyb;
        open[t] = op;
    }
    std::vector<int> tail(NT);
    for (int w = 0; w < NW; ++w) {
        int fbv[64], nf[64];
        for (int l = 0; l < 64; ++l) fbv[l] = first_bound[w * 64 + l] ? 1 : 0;
        dpp64(fbv, nf, WAVE_SHL1, 0);
        for (int l = 0; l < 64; ++l) {
            const int t = w * 64 + l;
            const bool holds_last = len[t] > 0 && t * c + len[t] == n;
            tail[t] = open[t] && (holds_last || (l != 63 && nf[l] != 0));
            g_inner_tails += tail[t] && !holds_last;
            count[t] += tail[t] ? 1 : 0;
        }
    }
    // 3. the run open at each chunk's start, and item offsets
    std::vector<NdFoldCarry> cin(NT), fin(NT);
    std::vector<int> cincl(NT), cex(NT);
    for (int w = 0; w < NW; ++w) {
        NdFoldCarry f[64], sh[64];
        int ci[64], cx[64];
        for (int l = 0; l < 64; ++l) {
            const int t = w * 64 + l;
            f[l] = NdFoldCarry{(any_bound[t] ? 1 : 0) | (len[t] > 0 && open[t] ? 2 : 0) | (runG[t] << 2),
                               runD[t]};
            ci[l] = count[t];
        }
        scan_carry64(f);
        dpp64(f, sh, WAVE_SHR1, NdFoldCarry{0, 0.0f});
        scan_int64(ci);
        dpp64(ci, cx, WAVE_SHR1, 0);
        for (int l = 0; l < 64; ++l) {
            fin[w * 64 + l] = f[l];
            cin[w * 64 + l] = sh[l];
            cincl[w * 64 + l] = ci[l];
            cex[w * 64 + l] = cx[l];
        }
    }
    std::vector<int> obase(NT, 0), lead(NT, 0);
    int total;
    if (NW > 1) {
        // each wave's carry-in, its lane 0's carried run, its item count,
        // from the per-wave values lane 63 (and lane 0) publish
        NdFoldCarry cw{0, 0.0f};
        total = 0;
        for (int k = 0; k < NW; ++k) {
            const int lk = k > 0 && first_bound[k * 64] && ((cw.flags >> 1) & 1) ? 1 : 0;
            for (int l = 0; l < 64; ++l) {
                const int t = k * 64 + l;
                cin[t] = then_h(cw, cin[t]);
                lead[t] = lk;
                obase[t] = total;
            }
            total += cincl[k * 64 + 63] + lk;
            g_leads += lk;
            cw = then_h(cw, fin[k * 64 + 63]);
        }
    } else {
        total = cincl[63];
    }
    if (total > kNdFoldItemsHost) return serial_fold(v, n);
    // 4. the items, each thread writing its own
    std::vector<float> items(size_t(total), std::nanf(""));
    std::vector<int> written(size_t(total), 0);
    auto put = [&](int o, float val) {
        if (o < 0 || o >= total) {
            std::fprintf(stderr, "item offset %d outside 0..%d\n", o, total);
            std::exit(3);
        }
        items[o] = val;
        ++written[o];
    };
    for (int t = 0; t < NT; ++t) {
        const int l = t & 63;
        int o = obase[t] + lead[t] + cex[t];
        if (l == 0 && lead[t]) put(obase[t], nd_fold_scale(cin[t].D, cin[t].flags >> 2));
        bool run = (cin[t].flags >> 1) & 1, runl = false;
        float D = run ? cin[t].D : 0.0f;
        int G = cin[t].flags >> 2;
        for (int j = 0; j < CMAX; ++j) {
            if (j < len[t]) {
                if ((inm[t] >> j) & 1u) {
                    D = run ? D + rr[size_t(t) * CMAX + j] : rr[size_t(t) * CMAX + j];
                    run = runl = true;
                    G = gg[size_t(t) * CMAX + j];
                } else {
                    if (runl) put(o++, nd_fold_scale(D, G));
                    put(o++, x[size_t(t) * CMAX + j]);
                    run = runl = false;
                }
            }
        }
        if (tail[t]) put(o, nd_fold_scale(D, G));
    }
    for (int k = 0; k < total; ++k)
        if (written[k] != 1) {
            std::fprintf(stderr, "item %d written %d times\n", k, written[k]);
            std::exit(3);
        }
    // 5. thread 0 folds them in order
    float s = 0.0f;
    for (int k = 0; k < total; ++k) s += items[k];
    items_out = items;
    *total_out = total;
    return s;
}

// The sequential item list for a given chunk prefix (the order the items
// must take), built one term after another.
std::vector<float> sequential_items(const float *a, int n, int nt, const std::vector<float> &excl)
{
    const int c = (n + nt - 1) / nt;
    std::vector<float> loc(n);
    for (int t = 0; t < nt; ++t) {
        float p = 0.0f;
        for (int j = 0; j < c && t * c + j < n; ++j) {
            p += a[t * c + j];
            loc[t * c + j] = p;
        }
    }
    const float dl = nd_fold_delta(n, c), cm = 1.0f - dl, cp = 1.0f + dl;
    std::vector<float> items;
    bool open = false;
    int openG = 0;
    float D = 0.0f;
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
                D = open ? D + r : r;
                open = true;
                openG = before;
            } else {
                if (open) items.push_back(nd_fold_scale(D, openG));
                open = false;
                items.push_back(a[i0 + j]);
            }
            before = after;
        }
    }
    if (open) items.push_back(nd_fold_scale(D, openG));
    return items;
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
    case 10:  // values from a tiny set, in a block of equal terms
        {
            const float base = float(1 + next_u64() % 7) * 0.125f * scale;
            for (auto &x : v) x = next_u64() % 8 ? base : base * 3.0f;
        }
        break;
    default:  // small terms in long runs, and a term as large as the running
              // sum (a binade crossing) on a wave's first or last chunk edge
        {
            const int nt = g_nt, c = (n + nt - 1) / nt;
            const float small = float(1 + next_u64() % 5) * 1e-3f * scale;
            for (auto &x : v) x = small * float(1 + next_u64() % 3);
            double s = 0.0;
            for (int i = 0; i < n; ++i) {
                const int edge = 64 * c;  // the first term of wave 1, 2, ...
                const int r = edge > 0 ? i % edge : 1;
                const int pick = int(g_edge_kind);
                const bool at = i > 0 && ((pick == 0 && r == 0) || (pick == 1 && r == edge - 1) ||
                                          (pick == 2 && (r == 0 || r == c)) ||
                                          (pick == 3 && r == edge - c));
                if (at) v[i] = float(s * (1.0 + unif()));
                s += v[i];
            }
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
    static const int threads[] = {256, 512, 256, 1024, 64, 128};
    // (threads, terms a thread): the device's instantiations (256 x 16 for
    // the softmax sums and row folds, 512 x 8 for the layer input's rms
    // norm, 256 x 12 for the other rms norms), a 16-wave form, the
    // single-wave form and a two-wave form
    static const int cmax_of[] = {16, 8, 12, 4, 32, 16};
    constexpr int kForms = sizeof(threads) / sizeof(threads[0]);
    int failures = 0;
    long long emulated = 0, cross_wave = 0;
    for (int kind = 0; kind <= 11; ++kind) {
        long long items = 0, runs = 0, bad = 0, fallback = 0;
        for (int k = 0; k < cases; ++k) {
            const int n = sizes[next_u64() % (sizeof(sizes) / sizeof(sizes[0]))];
            const int ti = int(next_u64() % kForms);
            const int nt = threads[ti];
            g_nt = nt;
            g_edge_kind = next_u64() % 4;
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
            // the device code lane for lane: its fold, and its items equal
            // in count and order to the sequential list for the same prefix
            std::vector<float> excl, dev_items;
            int total;
            const float dev = emulate_device(v.data(), n, nt, cmax_of[ti], excl, dev_items, &total);
            if (nd_f2u(dev) != nd_f2u(want)) {
                if (bad < 5)
                    std::printf("DEVICE MISMATCH kind %d n %d nt %d: got %a want %a\n", kind, n, nt, dev,
                                want);
                ++bad;
            }
            if (total >= 0) {
                ++emulated;
                const std::vector<float> seq = sequential_items(v.data(), n, nt, excl);
                bool same = int(seq.size()) == total;
                for (int q = 0; same && q < total; ++q) same = nd_f2u(seq[q]) == nd_f2u(dev_items[q]);
                if (!same) {
                    if (bad < 5)
                        std::printf("ITEMS kind %d n %d nt %d: device %d items, sequential %zu\n", kind, n,
                                    nt, total, seq.size());
                    ++bad;
                }
                if (nt > 64 && (n + nt - 1) / nt * 64 < n) ++cross_wave;
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
    std::printf("emulated %lld cases, %lld spanning waves, %lld lead items, %lld inner tails\n",
                emulated, cross_wave, g_leads, g_inner_tails);
    if (g_leads == 0 || g_inner_tails == 0) {
        std::printf("the generators never reached a wave-edge run\n");
        ++failures;
    }
    std::printf("%s\n", failures ? "FAIL" : "OK");
    return failures ? 1 : 0;
}
