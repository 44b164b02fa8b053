// The Needle-3 `.cact` container, read on the host and handed to the device
// model as canonical records (needle-infer/src/cact.rs, v3.rs).
//
//   header     49 little-endian u32 words, the last one rope_theta's bits
//   codebook   28 f32 (cb2 | cb3 | cb4, already scaled by 1/sqrt(group))
//   directory  one 44-byte record per tensor, no names: u8 dtype, u8 ndim,
//              u16 pad, u32 shape[4], u64 offset, u64 nbytes, u32 group,
//              u32 bits
//   blobs      64-byte aligned
//
// The directory is positional: the canon (embedding; per layer norm_in,
// q/k/v, the three conv taps when qkv_conv_taps > 0, q_norm, k_norm, gate,
// out, post_norm, attn_gate, pre_hada and the 13 HadamardMLP tensors; the six
// mHC scalars; phi_pre/post/res; the two Hadamard permutations; four tensors
// per Engram site; final_norm) is the only thing that says which record is
// which, so the slots the geometry fixes are shape-checked as the reference
// does before anything is uploaded.
#include "nd_cq_internal.h"
#include "nd_internal.h"

#include <algorithm>
#include <cstring>
#include <vector>

namespace {

constexpr uint32_t kTagV3 = 0x05E12A84u;  // cact.rs:31
constexpr size_t kHeaderV3 = 49 * 4;      // cact.rs:35
constexpr size_t kRecBytes = 44;          // cact.rs:37
constexpr size_t kCodebookLen = 28;       // cq::CODEBOOK_LEN
enum : uint8_t { kFp16 = 1, kFp32 = 2, kCq = 3, kRaw = 4 };

struct Rec {
    uint8_t dtype = 0, ndim = 0;
    size_t shape[4] = {0, 0, 0, 0};
    uint64_t offset = 0, nbytes = 0;
    size_t group = 0;
    uint8_t bits = 0;
};

struct Container {
    const uint8_t *raw = nullptr;
    size_t len = 0;
    nd_v3_cfg cfg{};
    std::vector<float> codebook;
    std::vector<Rec> recs;
    size_t canon = 0;  // records up to and including final_norm
    // canonical records for nd_v3_model_create, floats widened to f32
    std::vector<nd_v3_record> out;
    std::vector<std::vector<float>> floats;  // per canon record, its decoded floats
};

uint32_t le32(const uint8_t *p) { return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24; }
uint64_t le64(const uint8_t *p) { return uint64_t(le32(p)) | uint64_t(le32(p + 4)) << 32; }

// CactV3::from_bytes (cact.rs:994-1030), CactV3Geometry::from_words
// (cact.rs:345-393), parse_directory (cact.rs:423-480) and
// config_from_geometry (v3.rs:25-82), in that order of checks.
int parse(Container &c)
{
    if (c.len < kHeaderV3)
        return nd::fail(ND_ERR_CACT, "TooShort { need: %zu, got: %zu }", kHeaderV3, c.len);
    uint32_t w[49];
    for (int i = 0; i < 49; ++i) w[i] = le32(c.raw + 4 * i);
    if (w[0] != kTagV3) return nd::fail(ND_ERR_CACT, "BadTag(0x%08x)", w[0]);
    const size_t num_tensors = w[1], codebook_len = w[2];
    const size_t num_orders = w[26], num_sites = w[31];
    if (codebook_len != kCodebookLen)
        return nd::fail(ND_ERR_CACT, "BadCodebookLen(%zu)", codebook_len);
    const size_t dir_start = kHeaderV3 + codebook_len * 4;
    if (c.len < dir_start + num_tensors * kRecBytes)
        return nd::fail(ND_ERR_CACT, "TooShort { need: %zu, got: %zu }",
                        dir_start + num_tensors * kRecBytes, c.len);
    c.codebook.resize(codebook_len);
    for (size_t i = 0; i < codebook_len; ++i) {
        const uint32_t b = le32(c.raw + kHeaderV3 + 4 * i);
        std::memcpy(&c.codebook[i], &b, 4);
    }
    c.recs.resize(num_tensors);
    for (size_t i = 0; i < num_tensors; ++i) {
        const uint8_t *b = c.raw + dir_start + i * kRecBytes;
        Rec &r = c.recs[i];
        r.dtype = b[0];
        r.ndim = b[1];
        if (r.ndim > 4) return nd::fail(ND_ERR_CACT, "BadNdim { index: %zu, ndim: %u }", i, r.ndim);
        for (int k = 0; k < 4; ++k) r.shape[k] = le32(b + 4 + 4 * k);
        r.offset = le64(b + 20);
        r.nbytes = le64(b + 28);
        r.group = le32(b + 36);
        r.bits = uint8_t(le32(b + 40));
        const uint64_t end = r.nbytes > UINT64_MAX - r.offset ? UINT64_MAX : r.offset + r.nbytes;
        if (end > c.len)
            return nd::fail(ND_ERR_CACT,
                            "BlobOutOfRange { index: %zu, offset: %llu, nbytes: %llu, file: %zu }", i,
                            (unsigned long long)r.offset, (unsigned long long)r.nbytes, c.len);
    }

    // config_from_geometry
    nd_v3_cfg &g = c.cfg;
    g = nd_v3_cfg{};
    const size_t n_orders = num_orders < 4 ? num_orders : 4;
    const size_t n_sites = num_sites < 16 ? num_sites : 16;
    if (n_orders == 0) return nd::fail(ND_ERR_V3_GEOMETRY, "NoEngramOrders");
    const size_t tables = w[22], sub_dim = w[21], d_model = w[7];
    if (tables % n_orders != 0)
        return nd::fail(ND_ERR_V3_GEOMETRY, "TableCountNotDivisible { tables: %zu, orders: %zu }",
                        tables, n_orders);
    const size_t heads = tables / n_orders;
    const size_t derived = heads ? d_model / (n_orders * heads) : 0;
    if (heads == 0 || derived != sub_dim)
        return nd::fail(ND_ERR_V3_GEOMETRY, "SubDimMismatch { declared: %zu, derived: %zu }",
                        sub_dim, derived);
    if (w[9] == 0 || w[8] % w[9] != 0)
        return nd::fail(ND_ERR_V3_GEOMETRY, "HeadsNotDivisible { heads: %u, kv_heads: %u }", w[8],
                        w[9]);
    g.vocab_size = int32_t(w[5]);
    g.out_vocab = int32_t(w[6]);
    g.d_model = int32_t(w[7]);
    g.num_heads = int32_t(w[8]);
    g.num_kv_heads = int32_t(w[9]);
    g.num_layers = int32_t(w[10]);
    g.qk_head_dim = int32_t(w[11]);
    g.v_head_dim = int32_t(w[12]);
    g.max_seq_len = int32_t(w[13]);
    g.hada_n = int32_t(w[14]);
    g.mhc_lanes = int32_t(w[15]);
    g.sliding_window = int32_t(w[16]);
    const uint64_t global_mask = uint64_t(w[17]) | uint64_t(w[18]) << 32;
    for (uint32_t i = 0; i < w[10] && i < 64; ++i)
        if (global_mask >> i & 1) g.global_layers[g.n_global++] = int32_t(i);
    g.qkv_conv_taps = int32_t(w[19]);
    g.e_slots = int32_t(w[20]);
    g.e_sub_dim = int32_t(w[21]);
    g.e_heads = int32_t(heads);
    g.e_conv_taps = int32_t(w[23]);
    g.e_conv_dilation = int32_t(w[24]);
    g.e_seed_heads = int32_t(w[25]);
    g.n_orders = int32_t(n_orders);
    for (size_t k = 0; k < n_orders; ++k) g.orders[k] = int32_t(w[27 + k]);
    g.n_sites = int32_t(n_sites);
    for (size_t k = 0; k < n_sites; ++k) g.sites[k] = int32_t(w[32 + k]);
    std::memcpy(&g.rope_theta, &w[48], 4);
    return ND_OK;
}

// Canon positions (V3Layout::derive, v3.rs:236-330): the directory is
// positional, so slot s of layer li is record 1 + li * per_layer + s.
struct Canon {
    size_t per_layer, taps, layers_end, scalars, phi, perms, engram, final_norm, count;
    explicit Canon(const nd_v3_cfg &g)
    {
        taps = g.qkv_conv_taps > 0 ? 3 : 0;
        per_layer = 24 + taps;  // norm_in, q, k, v, [taps], q_norm, k_norm, gate, out,
                                // post_norm, attn_gate, pre_hada, 13 MLP tensors
        layers_end = 1 + size_t(g.num_layers) * per_layer;
        scalars = layers_end;
        phi = scalars + 6;
        perms = phi + 3;
        engram = perms + 2;
        final_norm = engram + 4 * size_t(g.n_sites);
        count = final_norm + 1;
    }
    size_t layer(int li, size_t slot) const { return 1 + size_t(li) * per_layer + slot; }
    // slot numbers within a layer
    size_t q(int li) const { return layer(li, 1); }
    size_t k(int li) const { return layer(li, 2); }
    size_t v(int li) const { return layer(li, 3); }
    size_t gate(int li) const { return layer(li, 6 + taps); }
    size_t out(int li) const { return layer(li, 7 + taps); }
    size_t attn_gate(int li) const { return layer(li, 9 + taps); }
};

// V3Layout::derive (the canon must fit the directory), validate (the slots
// the geometry fixes, v3.rs:336-386), then model_from_cact's reads in its
// order (v3.rs:438-482, layer_from_layout v3.rs:396-436): CQ slots must be
// CQ records (CactV3::cq, cact.rs:1076-1093; the blob itself is parsed by
// the device upload, CqWeight::from_blob), float slots are decoded
// (decode_floats, cact.rs:494-526).  With `kept` (a ladder rung), the shapes
// are still checked for every block but only the kept blocks and the Engram
// sites on them are read, in model_from_cact_at_depth's order
// (v3.rs:656-734): the embedding after the permutations.
int walk(Container &c, const std::vector<int> *kept = nullptr)
{
    const nd_v3_cfg &g = c.cfg;
    const size_t n = c.recs.size();
    const Canon cn(g);
    if (n < cn.count)
        return nd::fail(ND_ERR_V3_LAYOUT, "TooFewTensors { need: %zu, got: %zu }", n + 1, n);
    c.canon = cn.count;

    const size_t d = size_t(g.d_model);
    const size_t qd = size_t(g.num_heads) * g.qk_head_dim, kd = size_t(g.num_kv_heads) * g.qk_head_dim;
    const size_t vd = size_t(g.num_kv_heads) * g.v_head_dim, od = size_t(g.num_heads) * g.v_head_dim;
    const size_t nt = size_t(g.n_orders) * g.e_heads;
    auto shape = [&](size_t idx, const char *what, size_t w0, size_t w1) -> int {
        const Rec &r = c.recs[idx];
        if (r.shape[0] == w0 && r.shape[1] == w1) return ND_OK;
        return nd::fail(ND_ERR_V3_LAYOUT,
                        "BadShape { index: %zu, what: \"%s\", want: [%zu, %zu], got: [%zu, %zu] }",
                        idx, what, w0, w1, r.shape[0], r.shape[1]);
    };
    if (int rc = shape(0, "embedding", size_t(g.vocab_size), d)) return rc;
    for (int li = 0; li < g.num_layers; ++li) {
        if (int rc = shape(cn.q(li), "q_proj", qd, d)) return rc;
        if (int rc = shape(cn.k(li), "k_proj", kd, d)) return rc;
        if (int rc = shape(cn.v(li), "v_proj", vd, d)) return rc;
        if (int rc = shape(cn.gate(li), "gate_proj", od, d)) return rc;
        if (int rc = shape(cn.out(li), "out_proj", d, od)) return rc;
    }
    for (int s = 0; s < g.n_sites; ++s) {
        const size_t e = cn.engram + 4 * size_t(s);
        if (int rc = shape(e, "engram tables", nt * size_t(g.e_slots), size_t(g.e_sub_dim))) return rc;
        if (int rc = shape(e + 1, "engram key_proj", d, d)) return rc;
        if (int rc = shape(e + 2, "engram value_proj", d, d)) return rc;
    }

    c.out.assign(c.canon, nd_v3_record{});
    c.floats.resize(c.canon);
    auto cq = [&](size_t k) -> int {
        const Rec &r = c.recs[k];
        if (r.dtype != kCq)
            return nd::fail(ND_ERR_CACT, "DtypeMismatch { index: %zu, want: %u, got: %u }", k,
                            unsigned(kCq), unsigned(r.dtype));
        nd_v3_record &o = c.out[k];
        o.kind = ND_REC_CQ;
        o.data = c.raw + r.offset;
        o.len = size_t(r.nbytes);
        o.out = r.shape[0];
        o.in = r.shape[1];
        o.group = r.group;
        o.bits = r.bits;
        return ND_OK;
    };
    auto floats = [&](size_t k) -> int {
        const Rec &r = c.recs[k];
        std::vector<float> &v = c.floats[k];
        const uint8_t *b = c.raw + r.offset;
        if (r.dtype == kFp16) {
            if (r.nbytes % 2)
                return nd::fail(ND_ERR_CACT, "RaggedBlob { index: %zu, nbytes: %llu }", k,
                                (unsigned long long)r.nbytes);
            v.resize(size_t(r.nbytes / 2));
            for (size_t e = 0; e < v.size(); ++e)
                v[e] = nd_f16_to_f32(uint16_t(b[2 * e] | b[2 * e + 1] << 8));
        } else if (r.dtype == kFp32) {
            if (r.nbytes % 4)
                return nd::fail(ND_ERR_CACT, "RaggedBlob { index: %zu, nbytes: %llu }", k,
                                (unsigned long long)r.nbytes);
            v.resize(size_t(r.nbytes / 4));
            for (size_t e = 0; e < v.size(); ++e) {
                const uint32_t u = le32(b + 4 * e);
                std::memcpy(&v[e], &u, 4);
            }
        } else {
            return nd::fail(ND_ERR_CACT, "DtypeMismatch { index: %zu, want: %u, got: %u }", k,
                            unsigned(kFp16), unsigned(r.dtype));
        }
        nd_v3_record &o = c.out[k];
        o.kind = ND_REC_F32;
        o.data = v.data();
        o.len = v.size() * 4;
        o.out = r.ndim ? r.shape[0] : 1;
        o.in = r.ndim > 1 ? r.shape[1] : 1;
        return ND_OK;
    };
    auto on = [&](int li) {
        if (!kept) return true;
        for (int k : *kept)
            if (k == li) return true;
        return false;
    };
    if (!kept)
        if (int rc = cq(0)) return rc;
    for (int li = 0; li < g.num_layers; ++li) {
        if (!on(li)) continue;
        for (size_t t = 0; t < cn.taps; ++t)
            if (int rc = floats(cn.layer(li, 4 + t))) return rc;
        const size_t order[] = {0, 1, 2, 3, 4 + cn.taps, 5 + cn.taps, 6 + cn.taps, 7 + cn.taps,
                                8 + cn.taps, 9 + cn.taps, 10 + cn.taps};
        for (size_t slot : order) {
            const bool is_cq = slot >= 1 && slot <= 3 ? true : (slot == 6 + cn.taps || slot == 7 + cn.taps);
            if (int rc = is_cq ? cq(cn.layer(li, slot)) : floats(cn.layer(li, slot))) return rc;
        }
        // attn_gate is the first element of its tensor (v3.rs:415-418)
        nd_v3_record &ag = c.out[cn.attn_gate(li)];
        if (ag.len < 4)
            return nd::fail(ND_ERR_ARG, "EmptyScalar(\"attn_gate\") at record %zu", cn.attn_gate(li));
        ag.len = 4;
        ag.out = ag.in = 1;
        for (size_t m = 0; m < 13; ++m)
            if (int rc = floats(cn.layer(li, 11 + cn.taps + m))) return rc;
    }
    for (size_t k = 0; k < 6; ++k)
        if (int rc = floats(cn.scalars + k)) return rc;
    for (size_t k = 0; k < 3; ++k)
        if (int rc = cq(cn.phi + k)) return rc;
    for (int s = 0; s < g.n_sites; ++s) {
        if (!on(g.sites[s])) continue;
        const size_t e = cn.engram + 4 * size_t(s);
        if (int rc = cq(e)) return rc;
        if (int rc = cq(e + 1)) return rc;
        if (int rc = cq(e + 2)) return rc;
        if (int rc = floats(e + 3)) return rc;
    }
    for (size_t k = 0; k < 2; ++k)
        if (int rc = floats(cn.perms + k)) return rc;
    if (kept)
        if (int rc = cq(0)) return rc;
    return floats(cn.final_norm);
}

// ---- ladder rungs (v3/ladder.rs, v3.rs:612-734) -------------------------
// Every depth from 2 blocks up is a trained subnetwork of the full stack.  The
// blocks a rung keeps are a bisection from both ends: the order starts with
// the two endpoints and then repeatedly splits the widest remaining gap at its
// midpoint, the leftmost gap winning ties (ladder_order, ladder.rs:28-61); a
// rung of `depth` keeps the first `depth` of that order, ascending
// (ladder_layer_indices, ladder.rs:67-74).
std::vector<int> ladder_order(int L)
{
    std::vector<int> order;
    if (L <= 0) return order;
    if (L == 1) return {0};
    std::vector<int> sel = {0, L - 1};
    order = sel;
    while (int(order.size()) < L) {
        std::sort(sel.begin(), sel.end());
        int bg = 0, bl = 0, br = 0;
        for (size_t i = 0; i + 1 < sel.size(); ++i) {
            const int gap = sel[i + 1] - sel[i];
            if (gap <= 1) continue;
            if (gap > bg) {  // equal gaps keep the leftmost, met first
                bg = gap;
                bl = sel[i];
                br = sel[i + 1];
            }
        }
        if (bg == 0) break;
        const int mid = (bl + br) / 2;
        sel.push_back(mid);
        order.push_back(mid);
    }
    return order;
}

bool ladder_layers(int L, size_t depth, std::vector<int> &kept)
{
    if (depth < 2 || depth > size_t(L)) return false;
    const std::vector<int> order = ladder_order(L);
    kept.assign(order.begin(), order.begin() + std::ptrdiff_t(depth));
    std::sort(kept.begin(), kept.end());
    return true;
}

// config_at_depth (v3.rs:620-637): the kept blocks renumbered contiguously;
// global layers and Engram sites follow their blocks.
nd_v3_cfg config_at_depth(const nd_v3_cfg &p, const std::vector<int> &kept)
{
    nd_v3_cfg c = p;
    auto rank = [&](int l) {
        for (size_t i = 0; i < kept.size(); ++i)
            if (kept[i] == l) return int(i);
        return -1;
    };
    c.num_layers = int32_t(kept.size());
    c.n_global = 0;
    for (int i = 0; i < p.n_global; ++i)
        if (rank(p.global_layers[i]) >= 0) c.global_layers[c.n_global++] = rank(p.global_layers[i]);
    c.n_sites = 0;
    for (int i = 0; i < p.n_sites; ++i)
        if (rank(p.sites[i]) >= 0) c.sites[c.n_sites++] = rank(p.sites[i]);
    return c;
}

// The records of a rung, in the rung's own canon: the kept blocks whole, the
// per-layer mHC scalars and the phi lane rows of the kept blocks (Cactus-Quants
// packs each row on its own, so a row cut copies packed bytes and FP16 norms
// unchanged: CqWeight::select_rows, cq.rs:151-175), the Engram sites on kept
// blocks, the rest as is.  Nothing is re-quantised.
struct Rung {
    nd_v3_cfg cfg{};
    std::vector<nd_v3_record> out;
    std::vector<std::vector<float>> scalars;
    std::vector<std::vector<uint8_t>> phi;
};

int slice(const Container &c, const std::vector<int> &kept, Rung &r)
{
    const nd_v3_cfg &pg = c.cfg;
    r.cfg = config_at_depth(pg, kept);
    const Canon pc(pg), rc(r.cfg);
    const size_t n = size_t(pg.mhc_lanes), depth = kept.size();
    r.out.assign(rc.count, nd_v3_record{});
    r.out[0] = c.out[0];
    for (size_t i = 0; i < depth; ++i)
        for (size_t slot = 0; slot < pc.per_layer; ++slot)
            r.out[rc.layer(int(i), slot)] = c.out[pc.layer(kept[i], slot)];
    // a_pre, a_post, a_res: one per layer; b_pre, b_post: n; b_res: n * n
    const size_t width[6] = {1, 1, 1, n, n, n * n};
    r.scalars.resize(6);
    for (size_t k = 0; k < 6; ++k) {
        const std::vector<float> &v = c.floats[pc.scalars + k];
        std::vector<float> &o = r.scalars[k];
        for (int l : kept) {
            if ((size_t(l) + 1) * width[k] > v.size())
                return nd::fail(ND_ERR_ARG, "mHC scalar %zu is too short for layer %d", k, l);
            o.insert(o.end(), v.begin() + std::ptrdiff_t(size_t(l) * width[k]),
                     v.begin() + std::ptrdiff_t((size_t(l) + 1) * width[k]));
        }
        nd_v3_record rec = c.out[pc.scalars + k];
        rec.data = o.data();
        rec.len = o.size() * 4;
        rec.out = depth;
        r.out[rc.scalars + k] = rec;
    }
    // phi_pre, phi_post: rows l*n .. (l+1)*n; phi_res: rows l*n*n .. (l+1)*n*n
    const size_t rows[3] = {n, n, n * n};
    r.phi.resize(3);
    for (size_t k = 0; k < 3; ++k) {
        const nd_v3_record &src = c.out[pc.phi + k];
        if (src.group == 0 || src.group % 8 || (src.group & (src.group - 1)))
            return nd::fail(ND_ERR_ARG, "BadGroup(%zu) at record %zu", src.group, pc.phi + k);
        const size_t in_padded = (src.in + src.group - 1) / src.group * src.group;
        const size_t groups = in_padded / src.group;
        const size_t row_bytes = in_padded * (src.bits == 5 ? 2 : src.bits) / 8;
        const size_t packed = src.out * row_bytes, norms = src.out * groups * 2;
        if (src.len < packed + norms)
            return nd::fail(ND_ERR_ARG, "ShortBlob { need: %zu, got: %zu } at record %zu",
                            packed + norms, src.len, pc.phi + k);
        const uint8_t *b = static_cast<const uint8_t *>(src.data);
        std::vector<uint8_t> &o = r.phi[k];
        const size_t keep = depth * rows[k];
        o.resize(keep * (row_bytes + groups * 2));
        size_t at = 0;
        for (int pass = 0; pass < 2; ++pass)  // packed rows, then their norms
            for (int l : kept)
                for (size_t row = size_t(l) * rows[k]; row < (size_t(l) + 1) * rows[k]; ++row) {
                    if (row >= src.out) return nd::fail(ND_ERR_ARG, "mHC lane row out of range");
                    const size_t w = pass == 0 ? row_bytes : groups * 2;
                    std::memcpy(o.data() + at, b + (pass == 0 ? 0 : packed) + row * w, w);
                    at += w;
                }
        nd_v3_record rec = src;
        rec.data = o.data();
        rec.len = o.size();
        rec.out = keep;
        r.out[rc.phi + k] = rec;
    }
    for (size_t k = 0; k < 2; ++k) r.out[rc.perms + k] = c.out[pc.perms + k];
    size_t site = 0;
    for (int s = 0; s < pg.n_sites; ++s) {
        if (std::find(kept.begin(), kept.end(), pg.sites[s]) == kept.end()) continue;
        for (size_t k = 0; k < 4; ++k) r.out[rc.engram + 4 * site + k] = c.out[pc.engram + 4 * size_t(s) + k];
        ++site;
    }
    r.out[rc.final_norm] = c.out[pc.final_norm];
    return ND_OK;
}

// model_from_cact_at_depth's checks up to the slice (v3.rs:656-664): the
// parent geometry, the ladder, then the layout of the full container.
int read_rung(Container &c, const void *bytes, size_t len, size_t depth, std::vector<int> &kept)
{
    ND_REQUIRE(bytes || len == 0, "null container");
    c.raw = static_cast<const uint8_t *>(bytes);
    c.len = len;
    if (int rc = parse(c)) return rc;
    if (depth == size_t(c.cfg.num_layers)) {
        kept.clear();
        for (int l = 0; l < c.cfg.num_layers; ++l) kept.push_back(l);
        return walk(c);
    }
    if (!ladder_layers(c.cfg.num_layers, depth, kept))
        return nd::fail(ND_ERR_ARG, "depth is outside the ladder");
    return walk(c, &kept);
}

int read(Container &c, const void *bytes, size_t len)
{
    ND_REQUIRE(bytes || len == 0, "null container");
    c.raw = static_cast<const uint8_t *>(bytes);
    c.len = len;
    if (int rc = parse(c)) return rc;
    return walk(c);
}

}  // namespace

extern "C" {

int nd_v3_cact_config(const void *bytes, size_t len, nd_v3_cfg *cfg, size_t *canon_records)
{
    nd::clear_error();
    ND_REQUIRE(cfg, "null cfg");
    Container c;
    if (int rc = read(c, bytes, len)) return rc;
    *cfg = c.cfg;
    if (canon_records) *canon_records = c.canon;
    return ND_OK;
}

int nd_v3_model_from_cact(nd_ctx *ctx, const void *bytes, size_t len, nd_v3_model **out)
{
    ND_ENTER(ctx);
    ND_REQUIRE(out, "null output pointer");
    *out = nullptr;
    Container c;
    if (int rc = read(c, bytes, len)) return rc;
    return nd_v3_model_create(ctx, &c.cfg, c.codebook.data(), c.codebook.size(), c.out.data(),
                              c.out.size(), out);
}

size_t nd_v3_kv_bytes(const nd_v3_cfg *cfg, size_t seq_len, int kv_int8)
{
    nd::clear_error();
    if (!cfg) {
        nd::fail(ND_ERR_ARG, "cfg was null");
        return 0;
    }
    // V3Config::kv_bytes / kv_bytes_at (config.rs:143-179): per position a
    // key and a value per kv head, at 4 bytes, or at 1 byte plus an f32
    // scale for each; a local layer holds at most its window
    const size_t kvh = size_t(cfg->num_kv_heads);
    const size_t per = kvh * size_t(cfg->qk_head_dim + cfg->v_head_dim);
    const size_t per_pos = kv_int8 ? per + kvh * 8 : per * 4;
    size_t total = 0;
    for (int l = 0; l < cfg->num_layers; ++l) {
        bool global = cfg->sliding_window == 0;
        for (int g = 0; g < cfg->n_global && !global; ++g) global = cfg->global_layers[g] == l;
        const size_t slots = global ? seq_len : std::min(seq_len, size_t(cfg->sliding_window));
        total += slots * per_pos;
    }
    return total;
}

int nd_v3_ladder(size_t num_layers, size_t depth, int32_t *kept)
{
    nd::clear_error();
    ND_REQUIRE(kept, "null kept");
    ND_REQUIRE(num_layers <= 1024, "num_layers %zu too large", num_layers);
    std::vector<int> k;
    if (!ladder_layers(int(num_layers), depth, k)) return nd::fail(ND_ERR_ARG, "depth is outside the ladder");
    for (size_t i = 0; i < k.size(); ++i) kept[i] = k[i];
    return ND_OK;
}

int nd_v3_cact_config_at_depth(const void *bytes, size_t len, size_t depth, nd_v3_cfg *cfg,
                               int32_t *kept)
{
    nd::clear_error();
    ND_REQUIRE(cfg, "null cfg");
    Container c;
    std::vector<int> k;
    if (int rc = read_rung(c, bytes, len, depth, k)) return rc;
    *cfg = k.size() == size_t(c.cfg.num_layers) ? c.cfg : config_at_depth(c.cfg, k);
    if (kept)
        for (size_t i = 0; i < k.size(); ++i) kept[i] = k[i];
    return ND_OK;
}

int nd_v3_model_from_cact_at_depth(nd_ctx *ctx, const void *bytes, size_t len, size_t depth,
                                   nd_v3_model **out)
{
    ND_ENTER(ctx);
    ND_REQUIRE(out, "null output pointer");
    *out = nullptr;
    Container c;
    std::vector<int> k;
    if (int rc = read_rung(c, bytes, len, depth, k)) return rc;
    if (k.size() == size_t(c.cfg.num_layers))
        return nd_v3_model_create(ctx, &c.cfg, c.codebook.data(), c.codebook.size(), c.out.data(),
                                  c.out.size(), out);
    Rung r;
    if (int rc = slice(c, k, r)) return rc;
    return nd_v3_model_create(ctx, &r.cfg, c.codebook.data(), c.codebook.size(), r.out.data(),
                              r.out.size(), out);
}

}  // extern "C"
