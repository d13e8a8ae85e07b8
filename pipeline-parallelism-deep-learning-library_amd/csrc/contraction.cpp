// Contraction: C = alpha * A.B + beta * C over einsum labels, and the batched GEMM form.
//
// Host half of the contraction hot path. Follows the reference's planner
// (src/ops/contraction.rs) step for step where the semantics are observable:
//   * labels -> roles batch (A,B,C) / M (A,C) / N (B,C) / K (A,B)        (:344-442)
//   * gemm form: leading axes batch, last two M x K, K x N, M x N        (:444-494)
//   * per group: drop extent-1 axes, merge an axis into its slower neighbour when every
//     operand carrying it is contiguous, at most 4 strides per group     (:256-335)
//   * destination alias analysis (exact mixed-radix decode, hash set up to 2e6 elements,
//     conservative reject beyond)                                         (:518-662)
//   * plan Empty / Fill / Tiled / Split / General                         (:664-867)
// The MI355X parts are our own: the kernel geometry, the split-K sizing (targets two
// workgroups on each of 256 CUs, independent of the device so results are reproducible
// across boxes), the operand load modes, and 64-bit addressing (no u32 index limit).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <unordered_set>

#include "lg_internal.h"

namespace lg {
namespace {

constexpr uint64_t EXACT_LIMIT = 2000000;  // src/ops/contraction.rs:584
#ifndef LG_SPLIT_MIN_CHUNK
#define LG_SPLIT_MIN_CHUNK 128
#endif
constexpr uint32_t SPLIT_TARGET = 512;     // workgroups the split-K path aims for
constexpr uint32_t SPLIT_MIN_CHUNK = LG_SPLIT_MIN_CHUNK;  // K elements per split, at least
constexpr uint32_t SPLIT_MAX = 1024;

struct Axis {
    uint64_t extent = 1;
    bool ha = false, hb = false, hc = false;  // operand carries the axis
    uint64_t a = 0, b = 0, c = 0;             // its stride there
};

bool can_merge(const Axis& prev, const Axis& next) {
    auto ok = [&](bool hp, uint64_t sp, bool hn, uint64_t sn) {
        if (hp && hn) {
            if (sn != 0 && next.extent > UINT64_MAX / sn) return false;
            return sp == next.extent * sn;
        }
        return hp == hn;
    };
    return ok(prev.ha, prev.a, next.ha, next.a) && ok(prev.hb, prev.b, next.hb, next.b) &&
           ok(prev.hc, prev.c, next.hc, next.c);
}

Axis unit_axis(uint64_t extent) {
    Axis ax;
    ax.extent = extent;
    ax.ha = ax.hb = ax.hc = true;
    return ax;
}

// merge_group (src/ops/contraction.rs:278-312).
std::vector<Axis> merge_group(const std::vector<Axis>& axes, const char* group) {
    for (const Axis& ax : axes) {
        if (ax.extent == 0) return {unit_axis(0)};
    }
    std::vector<Axis> kept;
    for (const Axis& ax : axes) {
        if (ax.extent != 1) kept.push_back(ax);
    }
    if (kept.empty()) return {unit_axis(1)};
    std::vector<Axis> out{kept[0]};
    for (size_t i = 1; i < kept.size(); ++i) {
        const Axis& ax = kept[i];
        Axis& last = out.back();
        if (can_merge(last, ax)) {
            if (ax.extent != 0 && last.extent > UINT64_MAX / ax.extent) {
                fail_invalid(std::string(group) + " extent product overflows");
            }
            const uint64_t extent = last.extent * ax.extent;
            last = ax;
            last.extent = extent;
        } else {
            out.push_back(ax);
        }
    }
    if (out.size() > 4) {
        fail_invalid(std::string(group) + " group has " + std::to_string(out.size()) +
                     " strides after merging; the kernel supports 4");
    }
    return out;
}

struct Groups {
    std::vector<Axis> batch, m, n, k;
};

// parse_labels (src/ops/contraction.rs:344-355). One label per byte.
std::string parse_labels(const char* labels, size_t rank, const char* name) {
    if (labels == nullptr) fail_invalid(std::string("null labels for ") + name);
    std::string s(labels);
    if (s.size() != rank) {
        fail_invalid("label count " + std::to_string(s.size()) + " does not match rank " +
                     std::to_string(rank));
    }
    for (size_t i = 0; i < s.size(); ++i) {
        if (s.find(s[i]) != i) fail_invalid(std::string("repeated label '") + s[i] + "'");
    }
    return s;
}

enum class Role { Batch, M, N, K };

// groups_from_labels (src/ops/contraction.rs:380-442).
Groups groups_from_labels(const View& a, const std::string& la, const View& b,
                          const std::string& lb, const View& c, const std::string& lc) {
    std::string order;
    for (const std::string* ls : {&la, &lb, &lc}) {
        for (char ch : *ls) {
            if (order.find(ch) == std::string::npos) order.push_back(ch);
        }
    }
    struct Info {
        char label;
        Role role;
        Axis axis;
    };
    std::vector<Info> infos;
    for (char ch : order) {
        const size_t pa = la.find(ch), pb = lb.find(ch), pc = lc.find(ch);
        const bool fa = pa != std::string::npos, fb = pb != std::string::npos,
                   fc = pc != std::string::npos;
        Role role;
        if (fa && fb && fc) role = Role::Batch;
        else if (fa && !fb && fc) role = Role::M;
        else if (!fa && fb && fc) role = Role::N;
        else if (fa && fb && !fc) role = Role::K;
        else if (!fa && !fb && fc) fail_invalid(std::string("label '") + ch + "' appears only in C");
        else fail_invalid(std::string("label '") + ch + "' appears once");
        bool have = false;
        uint64_t extent = 1;
        auto see = [&](bool found, const View& v, size_t p) {
            if (!found) return;
            if (have && extent != v.shape[p]) {
                fail_invalid(std::string("extent mismatch for label '") + ch + "'");
            }
            have = true;
            extent = v.shape[p];
        };
        see(fa, a, pa);
        see(fb, b, pb);
        see(fc, c, pc);
        Axis ax;
        ax.extent = extent;
        ax.ha = fa;
        ax.hb = fb;
        ax.hc = fc;
        ax.a = fa ? a.strides[pa] : 0;
        ax.b = fb ? b.strides[pb] : 0;
        ax.c = fc ? c.strides[pc] : 0;
        infos.push_back({ch, role, ax});
    }
    auto take = [&](const std::string& labels, Role role) {
        std::vector<Axis> out;
        for (char ch : labels) {
            for (const Info& info : infos) {
                if (info.label == ch && info.role == role) out.push_back(info.axis);
            }
        }
        return out;
    };
    Groups g;
    g.batch = take(lc, Role::Batch);
    g.m = take(lc, Role::M);
    g.n = take(lc, Role::N);
    g.k = take(la, Role::K);
    return g;
}

// groups_from_gemm (src/ops/contraction.rs:444-494).
Groups groups_from_gemm(const View& a, const View& b, const View& c) {
    if (a.rank() < 2 || b.rank() < 2 || c.rank() < 2) fail_invalid("rank below 2");
    if (a.rank() != b.rank() || b.rank() != c.rank()) fail_invalid("ranks differ");
    const size_t r = a.rank();
    Groups g;
    for (size_t d = 0; d + 2 < r; ++d) {
        if (a.shape[d] != b.shape[d] || b.shape[d] != c.shape[d]) fail_invalid("batch extents differ");
        Axis ax;
        ax.extent = a.shape[d];
        ax.ha = ax.hb = ax.hc = true;
        ax.a = a.strides[d];
        ax.b = b.strides[d];
        ax.c = c.strides[d];
        g.batch.push_back(ax);
    }
    const uint64_t m = a.shape[r - 2], ka = a.shape[r - 1], kb = b.shape[r - 2], n = b.shape[r - 1];
    if (m != c.shape[r - 2] || n != c.shape[r - 1] || ka != kb) fail_invalid("inner extents differ");
    Axis am;
    am.extent = m;
    am.ha = am.hc = true;
    am.a = a.strides[r - 2];
    am.c = c.strides[r - 2];
    Axis an;
    an.extent = n;
    an.hb = an.hc = true;
    an.b = b.strides[r - 1];
    an.c = c.strides[r - 1];
    Axis ak;
    ak.extent = ka;
    ak.ha = ak.hb = true;
    ak.a = a.strides[r - 1];
    ak.b = b.strides[r - 2];
    g.m = {am};
    g.n = {an};
    g.k = {ak};
    return g;
}

// ---------------------------------------------------------------------------------------
// Destination alias analysis (src/ops/contraction.rs:496-662)
// ---------------------------------------------------------------------------------------
bool same_buffer(const View& a, const View& b) { return a.base == b.base; }

bool same_view(const View& a, const View& b) {
    return same_buffer(a, b) && a.offset == b.offset && a.shape == b.shape && a.strides == b.strides;
}

// Extent>1 axes sorted by ascending stride when they form a unique mixed-radix address.
bool decodable(const View& v, std::vector<std::pair<uint64_t, uint64_t>>* axes) {
    axes->clear();
    for (size_t d = 0; d < v.rank(); ++d) {
        if (v.shape[d] > 1) axes->push_back({v.shape[d], v.strides[d]});
    }
    std::stable_sort(axes->begin(), axes->end(),
                     [](const auto& x, const auto& y) { return x.second < y.second; });
    for (const auto& ax : *axes) {
        if (ax.second == 0) return false;
    }
    for (size_t i = 1; i < axes->size(); ++i) {
        const uint64_t extent = (*axes)[i - 1].first, stride = (*axes)[i - 1].second;
        if (extent != 0 && stride > UINT64_MAX / extent) return false;
        if ((*axes)[i].second < stride * extent) return false;
    }
    return true;
}

bool contains(const View& v, uint64_t elem, const std::vector<std::pair<uint64_t, uint64_t>>& asc) {
    if (elem < v.offset) return false;
    uint64_t rem = elem - v.offset;
    for (size_t i = asc.size(); i-- > 0;) {
        const uint64_t coord = rem / asc[i].second;
        if (coord >= asc[i].first) return false;
        rem -= coord * asc[i].second;
    }
    return rem == 0;
}

template <typename F>
void for_each_index(const View& v, F&& visit) {
    if (v.is_empty()) return;
    const size_t rank = v.rank();
    if (rank == 0) {
        visit(v.offset);
        return;
    }
    std::vector<uint64_t> idx(rank, 0);
    for (;;) {
        uint64_t e = v.offset;
        for (size_t d = 0; d < rank; ++d) e += idx[d] * v.strides[d];
        if (!visit(e)) return;
        size_t axis = rank - 1;
        for (;;) {
            if (++idx[axis] < v.shape[axis]) break;
            idx[axis] = 0;
            if (axis == 0) return;
            --axis;
        }
    }
}

bool shares(const View& a, const View& b) {
    if (!same_buffer(a, b)) return false;
    uint64_t a0, a1, b0, b1;
    if (!element_range(a, &a0, &a1) || !element_range(b, &b0, &b1)) return false;
    if (a0 >= b1 || b0 >= a1) return false;
    const bool a_small = a.len() <= b.len();
    const View& small = a_small ? a : b;
    const View& large = a_small ? b : a;
    std::vector<std::pair<uint64_t, uint64_t>> axes;
    bool hit = false;
    if (decodable(large, &axes)) {
        for_each_index(small, [&](uint64_t e) {
            hit = contains(large, e, axes);
            return !hit;
        });
        return hit;
    }
    // Unusual strides (or a stride of 0): exact for modest views, otherwise report overlap
    // rather than launch a kernel that would race.
    if (large.len() > EXACT_LIMIT) return true;
    std::unordered_set<uint64_t> seen;
    seen.reserve(large.len());
    for_each_index(large, [&](uint64_t e) {
        seen.insert(e);
        return true;
    });
    for_each_index(small, [&](uint64_t e) {
        hit = seen.count(e) != 0;
        return !hit;
    });
    return hit;
}

bool self_overlaps(const View& v) {
    std::vector<std::pair<uint64_t, uint64_t>> axes;
    if (v.len() <= 1 || decodable(v, &axes)) return false;
    if (v.len() > EXACT_LIMIT) return true;
    std::unordered_set<uint64_t> seen;
    seen.reserve(v.len());
    bool overlap = false;
    for_each_index(v, [&](uint64_t e) {
        if (!seen.insert(e).second) overlap = true;
        return !overlap;
    });
    return overlap;
}

void check_destination_alias(const View& a, const View& b, const View& c, uint64_t m, uint64_t n,
                             uint64_t k, bool reads_inputs) {
    if (self_overlaps(c)) fail_overlap("C writes the same element more than once");
    if (!reads_inputs) return;
    // In-place scale: C is A (or B) and every other extent is 1, so each output reads only
    // its own previous value. A and B may still alias each other.
    const bool inplace_a = k == 1 && n == 1 && same_view(c, a) && !shares(c, b);
    const bool inplace_b = k == 1 && m == 1 && same_view(c, b) && !shares(c, a);
    if (!inplace_a && (same_view(c, a) || shares(c, a))) fail_overlap("C overlaps A");
    if (!inplace_b && (same_view(c, b) || shares(c, b))) fail_overlap("C overlaps B");
}

// ---------------------------------------------------------------------------------------
// Planning
// ---------------------------------------------------------------------------------------
struct Merged {
    std::vector<Axis> batch, m, n, k;
    uint64_t batch_n = 1, m_n = 1, n_n = 1, k_n = 1;
};

uint64_t product(const std::vector<Axis>& axes) {
    uint64_t acc = 1;
    for (const Axis& ax : axes) {
        if (ax.extent != 0 && acc > UINT64_MAX / ax.extent) fail_invalid("dimension product overflows");
        acc *= ax.extent;
    }
    return acc;
}

Merged merge_all(const Groups& g) {
    Merged r;
    r.batch = merge_group(g.batch, "batch");
    r.m = merge_group(g.m, "M");
    r.n = merge_group(g.n, "N");
    r.k = merge_group(g.k, "K");
    r.batch_n = product(r.batch);
    r.m_n = product(r.m);
    r.n_n = product(r.n);
    r.k_n = product(r.k);
    return r;
}

uint32_t fit32(uint64_t x, const char* what) {
    if (x > 0x7fffffffull) {
        fail_invalid(std::string(what) + " " + std::to_string(x) +
                     " exceeds the kernels' 31-bit extent limit");
    }
    return static_cast<uint32_t>(x);
}

int64_t sfit(uint64_t x, const char* what) {
    if (x > static_cast<uint64_t>(INT64_MAX)) fail_invalid(std::string(what) + " too large");
    return static_cast<int64_t>(x);
}

Axes4 pack(const std::vector<Axis>& axes, char which) {
    Axes4 out;
    for (int i = 0; i < 4; ++i) {
        out.ext[i] = 1;
        out.stride[i] = 0;
    }
    const size_t n = axes.size();
    for (size_t i = 0; i < n; ++i) {
        const size_t slot = 4 - n + i;
        out.ext[slot] = fit32(axes[i].extent, "extent");
        const uint64_t s = which == 'a' ? axes[i].a : which == 'b' ? axes[i].b : axes[i].c;
        out.stride[slot] = sfit(s, "stride");
    }
    return out;
}

struct Plan {
    lg_contract_plan info{};
    bool half = false;  // f16 operands: the h* argument blocks below are the live ones
    GemmArgs gemm{};
    ReduceArgs reduce{};
    DotArgs dot{};
    GeneralArgs general{};
    FillArgs fill{};
    GemmHalfArgs hgemm{};
    GeneralHalfArgs hgeneral{};
    FillHalfArgs hfill{};
};

// 128-bit loads of eight halves need the view's first element 16-byte aligned and every other
// stride a multiple of eight elements.
int load_mode_half(uintptr_t base, uint64_t off, uint64_t sb, uint64_t srow, uint64_t sk) {
    auto al = [](uint64_t x) { return x % 8 == 0; };
    const bool start = (base + off * 2) % 16 == 0;
    if (sk == 1 && start && al(srow) && al(sb)) return LOAD_K;
    if (srow == 1 && start && al(sk) && al(sb)) return LOAD_MN;
    return LOAD_S;
}

// The f16 plans: the same kinds, on the f16 kernels. No split-K: one f64 tile per output block.
void plan_half(const View& a, const View& b, const View& c, const Merged& mg, float alpha,
               float beta, bool reads_inputs, Plan& p) {
    lg_contract_plan& info = p.info;
    p.half = true;
    uint16_t* cptr = reinterpret_cast<uint16_t*>(c.base) + c.offset;
    if (!reads_inputs) {
        info.kind = beta == 0.0f ? LG_PLAN_ZERO : LG_PLAN_SCALE;
        FillHalfArgs& f = p.hfill;
        f.c = cptr;
        f.count = mg.batch_n * mg.m_n * mg.n_n;
        f.m = fit32(mg.m_n, "M");
        f.n = fit32(mg.n_n, "N");
        f.batch = fit32(mg.batch_n, "batch");
        f.beta = beta;
        f.c_batch = pack(mg.batch, 'c');
        f.c_m = pack(mg.m, 'c');
        f.c_n = pack(mg.n, 'c');
        info.workgroups = (f.count + 255) / 256;
        return;
    }
    const uint32_t m = fit32(mg.m_n, "M"), n = fit32(mg.n_n, "N"), k = fit32(mg.k_n, "K"),
                   batch = fit32(mg.batch_n, "batch");
    const uint16_t* aptr = reinterpret_cast<const uint16_t*>(a.base) + a.offset;
    const uint16_t* bptr = reinterpret_cast<const uint16_t*>(b.base) + b.offset;
    const bool single = mg.batch.size() == 1 && mg.m.size() == 1 && mg.n.size() == 1 &&
                        mg.k.size() == 1;
    info.a_mode = LG_LOAD_STRIDED;
    info.b_mode = LG_LOAD_STRIDED;
    if (!single) {
        info.kind = LG_PLAN_GENERAL;
        GeneralHalfArgs& g = p.hgeneral;
        g.a = aptr;
        g.b = bptr;
        g.c = cptr;
        g.m = m;
        g.n = n;
        g.k = k;
        g.batch = batch;
        g.alpha = alpha;
        g.beta = beta;
        g.a_batch = pack(mg.batch, 'a');
        g.a_m = pack(mg.m, 'a');
        g.a_k = pack(mg.k, 'a');
        g.b_batch = pack(mg.batch, 'b');
        g.b_n = pack(mg.n, 'b');
        g.b_k = pack(mg.k, 'b');
        g.c_batch = pack(mg.batch, 'c');
        g.c_m = pack(mg.m, 'c');
        g.c_n = pack(mg.n, 'c');
        info.workgroups = (mg.batch_n * mg.m_n * mg.n_n + 255) / 256;
        return;
    }
    const Axis &ab = mg.batch[0], &am = mg.m[0], &an = mg.n[0], &ak = mg.k[0];
    GemmHalfArgs& t = p.hgemm;
    t.a = aptr;
    t.b = bptr;
    t.c = cptr;
    t.a_sb = sfit(ab.a, "A batch stride");
    t.a_sm = sfit(am.a, "A M stride");
    t.a_sk = sfit(ak.a, "A K stride");
    t.b_sb = sfit(ab.b, "B batch stride");
    t.b_sn = sfit(an.b, "B N stride");
    t.b_sk = sfit(ak.b, "B K stride");
    t.c_sb = sfit(ab.c, "C batch stride");
    t.c_sm = sfit(am.c, "C M stride");
    t.c_sn = sfit(an.c, "C N stride");
    t.m = m;
    t.n = n;
    t.k = k;
    t.batch = batch;
    t.tiles_m = (m + HGEMM_BM - 1) / HGEMM_BM;
    t.tiles_n = (n + HGEMM_BN - 1) / HGEMM_BN;
    info.tile_m = HGEMM_BM;
    info.tile_n = HGEMM_BN;
    info.a_mode = static_cast<uint32_t>(load_mode_half(a.base, a.offset, ab.a, am.a, ak.a));
    info.b_mode = static_cast<uint32_t>(load_mode_half(b.base, b.offset, ab.b, an.b, ak.b));
    t.alpha = alpha;
    t.beta = beta;
    const uint64_t wg = gemm_half_workgroups(m, n, batch);
    if (wg > 0x7fffffffull) fail_invalid("problem exceeds one launch's workgroup count");
    info.kind = LG_PLAN_TILED;
    info.workgroups = wg;
}

// (splits, k_chunk): one split when the output already fills the chip or K is short. The split
// count is capped so the partials (split_bytes each) fit in SPLIT_PARTIAL_MAX.
void split_shape(uint64_t tiles, uint32_t k, uint64_t split_bytes, uint32_t* splits,
                 uint32_t* chunk) {
    *splits = 1;
    *chunk = k;
    if (tiles >= SPLIT_TARGET / 2 || k < 2 * SPLIT_MIN_CHUNK) return;
    const uint64_t want = (SPLIT_TARGET + tiles - 1) / tiles;
    const uint64_t by_k = k / SPLIT_MIN_CHUNK;
    const uint64_t by_room = SPLIT_PARTIAL_MAX / split_bytes;
    const uint64_t rough = std::max<uint64_t>(1, std::min<uint64_t>({want, by_k, SPLIT_MAX, by_room}));
    uint64_t c = (k + rough - 1) / rough;
    c = (c + GEMM_BK - 1) / GEMM_BK * GEMM_BK;
    if (c == 0 || c >= k) return;
    *chunk = static_cast<uint32_t>(c);
    *splits = static_cast<uint32_t>((k + c - 1) / c);
}

// The same for 32x32 tiles of sixteen waves (gemm_f32_small): each split at least
// SMALL_SPLIT_CHUNK deep (one full batch of loads for every wave), SMALL_SPLIT_TARGET
// workgroups in all, one 1024-thread workgroup per compute unit (32x32 with K = 2^20:
// 512 workgroups 78 us, 256 68 us, 128 115 us).
constexpr uint32_t SMALL_SPLIT_CHUNK = 512;
constexpr uint32_t SMALL_SPLIT_TARGET = 256;
void small_split_shape(uint64_t tiles, uint32_t k, uint64_t split_bytes, uint32_t* splits,
                       uint32_t* chunk) {
    *splits = 1;
    *chunk = k;
    if (tiles >= SMALL_SPLIT_TARGET || k < 2 * SMALL_SPLIT_CHUNK) return;
    const uint64_t want = (SMALL_SPLIT_TARGET + tiles - 1) / tiles;
    const uint64_t rough = std::max<uint64_t>(
        1, std::min<uint64_t>({want, k / SMALL_SPLIT_CHUNK, SPLIT_MAX, SPLIT_PARTIAL_MAX / split_bytes}));
    uint64_t c = (k + rough - 1) / rough;
    c = (c + SMALL_SPLIT_CHUNK - 1) / SMALL_SPLIT_CHUNK * SMALL_SPLIT_CHUNK;
    if (c >= k) return;
    *chunk = static_cast<uint32_t>(c);
    *splits = static_cast<uint32_t>((k + c - 1) / c);
}

// The same for small outputs split along long K onto one-wave 32x32 direct-load tiles:
// SKINNY_SPLIT_TARGET workgroups in all (about four per compute unit, each with three 8 KB
// stages of loads in flight), each chunk at least SKINNY_MIN_CHUNK and a multiple of the
// 32-deep slice (32x32 with K = 2^20: 512 workgroups 68 us, 1024 51 us, 2048 51 us).
constexpr uint32_t SKINNY_SPLIT_TARGET = 1024;
constexpr uint32_t SKINNY_MIN_CHUNK = 256;
constexpr uint32_t SKINNY_BK = 32;
void skinny_split_shape(uint64_t tiles, uint32_t k, uint64_t split_bytes, uint32_t* splits,
                        uint32_t* chunk) {
    *splits = 1;
    *chunk = k;
    if (tiles >= SKINNY_SPLIT_TARGET || k < 2 * SKINNY_MIN_CHUNK) return;
    const uint64_t want = (SKINNY_SPLIT_TARGET + tiles - 1) / tiles;
    const uint64_t rough = std::max<uint64_t>(
        1, std::min<uint64_t>({want, k / SKINNY_MIN_CHUNK, SPLIT_MAX, SPLIT_PARTIAL_MAX / split_bytes}));
    uint64_t c = (k + rough - 1) / rough;
    c = (c + SKINNY_BK - 1) / SKINNY_BK * SKINNY_BK;
    if (c >= k) return;
    *chunk = static_cast<uint32_t>(c);
    *splits = static_cast<uint32_t>((k + c - 1) / c);
}

// The dot path's split: DOT_TARGET workgroups in all, each chunk at least DOT_MIN_CHUNK and a
// multiple of 1024 (four elements for each of 256 threads).
void dot_split_shape(uint32_t batch, uint32_t k, uint32_t* splits, uint32_t* chunk) {
    *splits = 1;
    *chunk = k;
    if (batch >= DOT_TARGET / 2 || k < 2 * DOT_MIN_CHUNK) return;
    const uint64_t want = (DOT_TARGET + batch - 1) / batch;
    const uint64_t rough = std::max<uint64_t>(
        1, std::min<uint64_t>({want, k / DOT_MIN_CHUNK, SPLIT_PARTIAL_MAX / (4ull * batch)}));
    uint64_t c = (k + rough - 1) / rough;
    c = (c + 1023) / 1024 * 1024;
    if (c >= k) return;
    *chunk = static_cast<uint32_t>(c);
    *splits = static_cast<uint32_t>((k + c - 1) / c);
}

// Compute units of one MI355X, for the tile-size choice only.
constexpr uint64_t GEMM_CUS = 256;
// K elements per chunk below which two wave groups would each get too few slices to pipeline.
constexpr uint32_t KG_MIN_CHUNK = 256;
// Longest K for which 64x64 tiles replace a split 128x128 grid.
constexpr uint32_t FILLS64_MAX_K = 4096;

// Waves a many-tile 32x32 product needs before it takes one tile per wave (gemm_f32_wave)
// rather than sixteen waves per tile (gemm_f32_small).
constexpr uint64_t WAVE_MIN_TILES = 1024;

// 128-bit loads need the view's first element 16-byte aligned (allocation base included) and
// every other stride a multiple of four elements.
int load_mode(uintptr_t base, uint64_t off, uint64_t sb, uint64_t srow, uint64_t sk) {
    auto al = [](uint64_t x) { return x % 4 == 0; };
    const bool start = (base + off * sizeof(float)) % 16 == 0;
    if (sk == 1 && start && al(srow) && al(sb)) return LOAD_K;
    if (srow == 1 && start && al(sk) && al(sb)) return LOAD_MN;
    return LOAD_S;
}

Plan plan_merged(const View& a, const View& b, const View& c, const Merged& mg, float alpha,
                 float beta, bool half) {
    Plan p;
    lg_contract_plan& info = p.info;
    info.batch = mg.batch_n;
    info.m = mg.m_n;
    info.n = mg.n_n;
    info.k = mg.k_n;
    info.splits = 1;
    info.k_chunk = mg.k_n;
    info.kgroups = 1;
    info.groups = static_cast<uint32_t>(
        std::max({mg.batch.size(), mg.m.size(), mg.n.size(), mg.k.size()}));
    if (mg.m_n == 0 || mg.n_n == 0 || mg.batch_n == 0) {
        info.kind = LG_PLAN_EMPTY;
        return p;
    }
    const bool reads_inputs = alpha != 0.0f && mg.k_n != 0;
    check_destination_alias(a, b, c, mg.m_n, mg.n_n, mg.k_n, reads_inputs);
    if (half) {
        plan_half(a, b, c, mg, alpha, beta, reads_inputs, p);
        return p;
    }
    float* cptr = reinterpret_cast<float*>(c.base) + c.offset;
    if (!reads_inputs) {
        info.kind = beta == 0.0f ? LG_PLAN_ZERO : LG_PLAN_SCALE;
        FillArgs& f = p.fill;
        f.c = cptr;
        f.count = mg.batch_n * mg.m_n * mg.n_n;
        f.m = fit32(mg.m_n, "M");
        f.n = fit32(mg.n_n, "N");
        f.batch = fit32(mg.batch_n, "batch");
        f.beta = beta;
        f.c_batch = pack(mg.batch, 'c');
        f.c_m = pack(mg.m, 'c');
        f.c_n = pack(mg.n, 'c');
        info.workgroups = (f.count + 255) / 256;
        return p;
    }
    const uint32_t m = fit32(mg.m_n, "M"), n = fit32(mg.n_n, "N"), k = fit32(mg.k_n, "K"),
                   batch = fit32(mg.batch_n, "batch");
    const float* aptr = reinterpret_cast<const float*>(a.base) + a.offset;
    const float* bptr = reinterpret_cast<const float*>(b.base) + b.offset;
    const bool single = mg.batch.size() == 1 && mg.m.size() == 1 && mg.n.size() == 1 &&
                        mg.k.size() == 1;
    // The tiled kernel scales A by alpha as it stages it; with a non-finite alpha its zero
    // padding would become NaN, so such calls take the general kernel, which reads real
    // elements only.
    if (!single || !std::isfinite(alpha)) {
        info.kind = LG_PLAN_GENERAL;
        GeneralArgs& g = p.general;
        g.a = aptr;
        g.b = bptr;
        g.c = cptr;
        g.m = m;
        g.n = n;
        g.k = k;
        g.batch = batch;
        g.alpha = alpha;
        g.beta = beta;
        g.a_batch = pack(mg.batch, 'a');
        g.a_m = pack(mg.m, 'a');
        g.a_k = pack(mg.k, 'a');
        g.b_batch = pack(mg.batch, 'b');
        g.b_n = pack(mg.n, 'b');
        g.b_k = pack(mg.k, 'b');
        g.c_batch = pack(mg.batch, 'c');
        g.c_m = pack(mg.m, 'c');
        g.c_n = pack(mg.n, 'c');
        info.workgroups = (mg.batch_n * mg.m_n * mg.n_n + 255) / 256;
        return p;
    }
    const Axis &ab = mg.batch[0], &am = mg.m[0], &an = mg.n[0], &ak = mg.k[0];
    if (m == 1 && n == 1) {
        // Dot products: memory-bound, summed on the VALU.
        DotArgs& d = p.dot;
        d.a = aptr;
        d.b = bptr;
        d.c = cptr;
        d.a_sb = sfit(ab.a, "A batch stride");
        d.a_sk = sfit(ak.a, "A K stride");
        d.b_sb = sfit(ab.b, "B batch stride");
        d.b_sk = sfit(ak.b, "B K stride");
        d.c_sb = sfit(ab.c, "C batch stride");
        d.k = k;
        d.batch = batch;
        d.alpha = alpha;
        d.beta = beta;
        d.scale_b = 0;
        uint32_t splits = 1, chunk = k;
        dot_split_shape(batch, k, &splits, &chunk);
        if (static_cast<uint64_t>(batch) * splits > 0x7fffffffull) {
            fail_invalid("problem exceeds one launch's workgroup count");
        }
        d.splits = splits;
        d.k_chunk = chunk;
        const bool vec = ak.a == 1 && ak.b == 1 && ab.a % 4 == 0 && ab.b % 4 == 0 &&
                         (a.base + a.offset * sizeof(float)) % 16 == 0 &&
                         (b.base + b.offset * sizeof(float)) % 16 == 0;
        info.kind = LG_PLAN_DOT;
        info.kernel = LG_KERNEL_DOT;
        info.a_mode = info.b_mode = vec ? LG_LOAD_K_CONTIG : LG_LOAD_STRIDED;
        info.tile_m = info.tile_n = 1;
        info.splits = splits;
        info.k_chunk = chunk;
        info.workgroups = static_cast<uint64_t>(batch) * splits;
        info.scratch_bytes = splits > 1 ? static_cast<uint64_t>(batch) * splits * sizeof(float) : 0;
        return p;
    }
    // Operand roles. C contiguous along M (and not along N) is computed as C^T = B^T.A^T, so
    // the epilogue's stores run along C's unit stride; alpha then multiplies the operand loaded
    // as B (the caller's A), and every product is still (alpha*a)*b.
    struct Role {
        const float* ptr;
        uintptr_t base;
        uint64_t offset, sb, srow, sk;
    };
    Role ra{aptr, a.base, a.offset, ab.a, am.a, ak.a};
    Role rb{bptr, b.base, b.offset, ab.b, an.b, ak.b};
    uint64_t c_sm = am.c, c_sn = an.c;
    const bool swap = am.c == 1 && an.c != 1;
    uint32_t mm = m, nn = n;
    if (swap) {
        std::swap(ra, rb);
        std::swap(c_sm, c_sn);
        std::swap(mm, nn);
    }
    info.swapped = swap ? 1 : 0;
    GemmArgs& t = p.gemm;
    t.a = ra.ptr;
    t.b = rb.ptr;
    t.c = cptr;
    t.partial = nullptr;
    t.a_sb = sfit(ra.sb, "A batch stride");
    t.a_sm = sfit(ra.srow, "A M stride");
    t.a_sk = sfit(ra.sk, "A K stride");
    t.b_sb = sfit(rb.sb, "B batch stride");
    t.b_sn = sfit(rb.srow, "B N stride");
    t.b_sk = sfit(rb.sk, "B K stride");
    t.c_sb = sfit(ab.c, "C batch stride");
    t.c_sm = sfit(c_sm, "C M stride");
    t.c_sn = sfit(c_sn, "C N stride");
    t.m = mm;
    t.n = nn;
    t.k = k;
    t.batch = batch;
    t.alpha = alpha;
    t.beta = beta;
    t.scale_b = swap ? 1 : 0;
    if (k <= OUTER_MAX_K) {
        // Low-rank updates (rank-1 and the like): memory-bound on C, on the VALU in the
        // reference's own order, four outputs per thread.
        auto al = [](uint64_t x) { return x % 4 == 0; };
        t.kernel = KERN_OUTER;
        t.tile = 1;
        t.tile_n = 4;
        t.splits = 1;
        t.k_chunk = k;
        t.tiles_m = mm;
        t.tiles_n = (nn + 3) / 4;
        t.vec_c = c_sn == 1 && al(nn) && al(c_sm) && al(ab.c) && (c.base + c.offset * 4) % 16 == 0;
        t.vec_b = rb.srow == 1 && al(nn) && al(rb.sk) && al(rb.sb) &&
                  (rb.base + rb.offset * 4) % 16 == 0;
        info.kind = LG_PLAN_TILED;
        info.kernel = LG_KERNEL_OUTER;
        info.tile_m = 1;
        info.tile_n = 4;
        info.a_mode = LG_LOAD_STRIDED;
        info.b_mode = t.vec_b ? LG_LOAD_MN_CONTIG : LG_LOAD_STRIDED;
        info.workgroups = gemm_workgroups(t);
        return p;
    }
    // Tile choice. 128x128 tiles load half the operand bytes per product of 64x64 ones, so they
    // are kept whenever at least half of their area is output and their grid, split along K as
    // far as split_shape would go, reaches GEMM_SMALL_BELOW workgroups; otherwise 64x64 tiles
    // give four times the workgroups before split-K adds more. Outputs that even 64x64 tiles
    // would pad past half (batches of small matrices, skinny outputs) take 32x32 tiles: one per
    // wave when there are enough of them, else sixteen waves per tile splitting K.
    auto grid_of = [&](uint32_t e) {
        return static_cast<uint64_t>((mm + e - 1) / e) * ((nn + e - 1) / e) * batch;
    };
    const uint64_t useful = static_cast<uint64_t>(mm) * nn * batch;
    const uint64_t big = grid_of(GEMM_BM), mid = grid_of(GEMM_SMALL_TILE), tiny = grid_of(GEMM_TINY_TILE);
    const uint64_t k_ways = std::max<uint64_t>(1, std::min<uint64_t>(k / SPLIT_MIN_CHUNK, SPLIT_MAX));
    if (mid < GEMM_SMALL_BELOW && k <= GEMM_SMALL_K) {
        t.tile = GEMM_TINY_TILE;  // one launch, no split-K partials
        t.kernel = KERN_SMALL;
    } else if (2 * useful >= big * GEMM_BM * GEMM_BN) {
        // A compute unit's time follows the tiles it holds (four 128x128 workgroups share one
        // at a time), and a 64x64 tile is a quarter of the work at ~0.85 of the efficiency, so
        // 64x64 tiles also win when the 128x128 grid spreads unevenly over the chip's
        // GEMM_CUS compute units (2304^3: 324 tiles, 312 -> 272 us) but not when it spreads
        // evenly (2048^3: 256 tiles, 172 vs 177 us). Grids under GEMM_CUS tiles split along K
        // instead. The constant is the part's; plans depend on the shape alone.
        const uint64_t rounds_big = (big + GEMM_CUS - 1) / GEMM_CUS;
        const uint64_t rounds_mid = (mid + GEMM_CUS - 1) / GEMM_CUS;
        const bool uneven = big >= GEMM_CUS && 20 * rounds_mid < 68 * rounds_big;
        // A 128x128 grid that would need split-K to fill the chip takes 64x64 tiles when those
        // alone fill it in (nearly) whole rounds and K is short, so the split chunks would be
        // only a few slices deep (1024^3: 64 tiles split 8 ways, 54 TFLOP/s; 256 64x64 tiles,
        // 73; 1024x2048x1024: 75 -> 89). Otherwise the split grid balances better (1280^3, 400
        // 64x64 tiles: 71 against 80; 1536^3: 79 against 87; 1536^2 x 65536: 83 against 110).
        const uint64_t rounds64 = (mid + GEMM_CUS - 1) / GEMM_CUS;
        const bool fills64 = big < GEMM_CUS && mid >= GEMM_CUS && 10 * mid >= 9 * rounds64 * GEMM_CUS &&
                             k <= FILLS64_MAX_K;
        t.tile = big * k_ways < GEMM_SMALL_BELOW || uneven || fills64 ? GEMM_SMALL_TILE : GEMM_BM;
        t.kernel = KERN_TILE;
    } else if (2 * useful >= mid * GEMM_SMALL_TILE * GEMM_SMALL_TILE) {
        t.tile = GEMM_SMALL_TILE;
        t.kernel = KERN_TILE;
    } else {
        t.tile = GEMM_TINY_TILE;
        t.kernel = tiny >= WAVE_MIN_TILES ? KERN_WAVE : KERN_SMALL;
    }
    const int a_mode = load_mode(ra.base, ra.offset, ra.sb, ra.srow, ra.sk);
    const int b_mode = load_mode(rb.base, rb.offset, rb.sb, rb.srow, rb.sk);
    info.a_mode = static_cast<uint32_t>(a_mode);
    info.b_mode = static_cast<uint32_t>(b_mode);
    t.tile_n = t.tile;
    if (t.kernel == KERN_TILE && t.tile == GEMM_BM && a_mode != LOAD_S && b_mode != LOAD_S) {
        // Both operands have a 16-byte aligned unit-stride axis: slices go straight into LDS.
        // 128x256 tiles (eight waves, two workgroups per compute unit) when at least
        // 2 * GEMM_CUS of them fill the chip in whole rounds (4096^3: 131 -> 137 TFLOP/s,
        // config 5 131 -> 138); otherwise 128x128 tiles, three workgroups per compute unit,
        // also for split-K.
        t.kernel = KERN_DIRECT;
        const uint64_t wide = static_cast<uint64_t>((mm + GEMM_BM - 1) / GEMM_BM) *
                              ((nn + GEMM_WIDE_N - 1) / GEMM_WIDE_N) * batch;
        if (wide >= 2 * GEMM_CUS) t.tile_n = GEMM_WIDE_N;
    }
    t.tiles_m = (mm + t.tile - 1) / t.tile;
    t.tiles_n = (nn + t.tile_n - 1) / t.tile_n;
    info.tile_m = t.tile;
    info.tile_n = t.tile_n;
    const uint64_t tiles = static_cast<uint64_t>(t.tiles_m) * t.tiles_n * batch;
    const uint64_t split_bytes = static_cast<uint64_t>(batch) * mm * nn * sizeof(float);
    uint32_t splits = 1, chunk = k;
    if (t.kernel == KERN_TILE || t.kernel == KERN_DIRECT) {
        split_shape(tiles, k, split_bytes, &splits, &chunk);
    } else if (t.kernel == KERN_SMALL && !(mid < GEMM_SMALL_BELOW && k <= GEMM_SMALL_K)) {
        // Small outputs with long K. Whole 32x32 tiles whose operands both have a 16-byte
        // aligned unit-stride axis go to one-wave direct-load tiles when the split fills the
        // chip: their loads read 8 rows x 128 B per wave instruction, where the sixteen-wave
        // kernel's go straight to MFMA registers at 32 rows x 32 B (32x32 with K = 2^20: 68 ->
        // 51 us). Other outputs keep the sixteen-wave kernel.
        uint32_t ds = 1, dc = k;
        const bool whole = mm % GEMM_TINY_TILE == 0 && nn % GEMM_TINY_TILE == 0;
        if (whole && a_mode != LOAD_S && b_mode != LOAD_S) {
            skinny_split_shape(tiles, k, split_bytes, &ds, &dc);
        }
        if (ds > 1 && tiles * ds >= GEMM_CUS) {
            t.kernel = KERN_DIRECT;
            splits = ds;
            chunk = dc;
        } else {
            small_split_shape(tiles, k, split_bytes, &splits, &chunk);
        }
    }
    if (tiles * splits > 0x7fffffffull) fail_invalid("problem exceeds one launch's workgroup count");
    // Grids that leave at most one workgroup per compute unit (four waves, one per SIMD) run
    // several wave groups per workgroup on consecutive parts of each K chunk, so every SIMD has
    // more waves to issue MFMAs while one waits: 128x128 direct-load tiles two groups of
    // 32-deep slices in two stages (2048^3: 107 -> 119 TFLOP/s; three groups 117, four 112),
    // 64x64 tiles with aligned operands four groups of 32-deep slices on the direct-load
    // kernel (1024^3: 68 -> 77).
    t.kgroups = 1;
    if (tiles * splits <= GEMM_CUS) {
        if (t.kernel == KERN_DIRECT && t.tile == GEMM_BM && t.tile_n == GEMM_BN &&
            chunk >= KG_MIN_CHUNK) {
            t.kgroups = 2;
        } else if (t.kernel == KERN_TILE && t.tile == GEMM_SMALL_TILE && a_mode != LOAD_S &&
                   b_mode != LOAD_S && chunk >= 2 * KG_MIN_CHUNK) {
            t.kernel = KERN_DIRECT;
            t.kgroups = 4;
        }
    }
    // Full 128x128 tiles with K chunks in whole pipeline steps take the software-pipelined
    // kernel: with at least two workgroups per compute unit on 16-deep slices, 128x128 tiles
    // also where 128x256 ones were chosen (4096^3: 137 -> 142.5 TFLOP/s; config 3 134 -> 137;
    // config 4 106 -> 112; config 5 137.5 -> 143), and 32-deep slices for (K, K) operands with
    // chunks of at least PIPE_DEEP_K (config 5's dX: 140 -> 145); with one workgroup per compute
    // unit on 32-deep slices, in place of two wave groups (2048^3: 119 -> 135).
    t.slice_k = 0;
    const uint32_t last_chunk = k - (splits - 1) * chunk;
    const bool full = mm % GEMM_BM == 0 && nn % GEMM_BN == 0;
    auto whole = [&](uint32_t bk) {
        return chunk % (PIPE_STAGES * bk) == 0 && last_chunk % (PIPE_STAGES * bk) == 0;
    };
    const uint64_t tiles128 = full ? static_cast<uint64_t>(mm / GEMM_BM) * (nn / GEMM_BN) * batch * splits : 0;
    // Full 64x64 tiles that would run four wave groups sharing stages instead take four waves
    // with a quarter of K each, no barrier in the loop (1024^3: 75 -> 97-99 TFLOP/s).
    const bool full64 = mm % GEMM_SMALL_TILE == 0 && nn % GEMM_SMALL_TILE == 0;
    if (t.kernel == KERN_DIRECT && t.tile == GEMM_SMALL_TILE && t.kgroups == 4 && full64 &&
        chunk % KW_STEP == 0 && last_chunk % KW_STEP == 0) {
        t.kernel = KERN_PIPE;
        t.slice_k = KW_BK;
    }
    if (t.kernel == KERN_DIRECT && t.tile == GEMM_BM && full) {
        if (t.kgroups == 1 && tiles128 >= 2 * GEMM_CUS && whole(16)) {
            const bool deep = a_mode == LOAD_K && b_mode == LOAD_K && chunk >= PIPE_DEEP_K && whole(32);
            t.slice_k = deep ? 32 : 16;
        } else if (t.kgroups == 2 && whole(32)) {
            t.slice_k = 32;
            t.kgroups = 1;
        }
        if (t.slice_k != 0) {
            t.kernel = KERN_PIPE;
            t.tile_n = GEMM_BN;
            t.tiles_n = nn / GEMM_BN;
            info.tile_n = GEMM_BN;
        }
    }
    // Grids of 128x64 tiles that fill three workgroups per compute unit in one round (more
    // than 2 * GEMM_CUS, at most 3 * GEMM_CUS), where 128x128 tiles would leave many compute
    // units with one tile and others with two: 128x64 tiles on the pipelined kernel, three
    // workgroups per compute unit (the rank-4 48^6 product, 2304^3: 324 tiles of 128x128 or
    // 648 of 128x64; 97 -> 116 TFLOP/s against 64x64 tiles).
    const uint64_t tiles_n64 = static_cast<uint64_t>(mm / GEMM_BM) * (nn / PIPE_NARROW_N) * batch;
    if ((t.kernel == KERN_DIRECT || t.kernel == KERN_TILE) && t.slice_k == 0 && t.kgroups == 1 &&
        splits == 1 && a_mode != LOAD_S && b_mode != LOAD_S && mm % GEMM_BM == 0 &&
        nn % PIPE_NARROW_N == 0 && chunk % (PIPE_STAGES * 16) == 0 && tiles_n64 > 2 * GEMM_CUS &&
        tiles_n64 <= 3 * GEMM_CUS) {
        t.kernel = KERN_PIPE;
        t.slice_k = 16;
        t.tile = GEMM_BM;
        t.tile_n = PIPE_NARROW_N;
        t.tiles_m = mm / GEMM_BM;
        t.tiles_n = nn / PIPE_NARROW_N;
        info.tile_m = GEMM_BM;
        info.tile_n = PIPE_NARROW_N;
    }
    // Split-K products of at most GEMM_CUS / 2 full 64x64 tiles (short outputs, long K) take the
    // K-split-wave kernel on 64x64 tiles instead, split to about one workgroup per compute unit
    // in chunks of whole steps: fewer, longer splits (config 4: 16 of 4096 instead of 128 of
    // 512 on 128x128 tiles, 4 MiB of partials instead of 32; 112 -> 116 TFLOP/s).
    const uint32_t kw_step = KW_STEP;
    if (t.kernel == KERN_PIPE && t.tile == GEMM_BM && splits > 1 && full64 && k % kw_step == 0) {
        const uint64_t t64 = static_cast<uint64_t>(mm / GEMM_SMALL_TILE) * (nn / GEMM_SMALL_TILE) * batch;
        if (t64 <= GEMM_CUS / 2) {
            uint64_t s64 = GEMM_CUS / t64;
            const uint64_t c64 = ((k + s64 - 1) / s64 + kw_step - 1) / kw_step * kw_step;
            s64 = (k + c64 - 1) / c64;
            if (s64 > 1 && s64 * split_bytes <= SPLIT_PARTIAL_MAX) {
                t.tile = t.tile_n = GEMM_SMALL_TILE;
                t.tiles_m = mm / GEMM_SMALL_TILE;
                t.tiles_n = nn / GEMM_SMALL_TILE;
                info.tile_m = info.tile_n = GEMM_SMALL_TILE;
                splits = static_cast<uint32_t>(s64);
                chunk = static_cast<uint32_t>(c64);
                t.kgroups = PIPE_KW;
                t.slice_k = KW_BK;
            }
        }
    }
    // Full 128x128 pipelined tiles on 16-deep slices (grids of at least two workgroups per
    // compute unit) with A contiguous along K pair up along M into 256x128 tiles of eight waves
    // (gemm_f32_pl256, one workgroup per compute unit): the same waves, 3/4 of the operand
    // loads (4096^3: 142 -> 144-145 TFLOP/s, config 3 134 -> 136-138, config 5's Y 143 -> 145).
    // A contiguous along M keeps 128x128 tiles (config 5's dW: 138 against 135).
    if (t.kernel == KERN_PIPE && t.tile == GEMM_BM && t.tile_n == GEMM_BN && t.slice_k == 16 &&
        splits == 1 && a_mode == LOAD_K && mm % PIPE_TALL_M == 0 && k % (PIPE_STAGES * 16) == 0) {
        t.tile = PIPE_TALL_M;
        t.tiles_m = mm / PIPE_TALL_M;
        info.tile_m = PIPE_TALL_M;
    }
    // Full 256x256 tiles, at least one per compute unit, whose A-role operand is contiguous
    // along K take eight waves of 4x2 blocks (gemm_f32_pl2x, one workgroup per compute unit):
    // per FLOP 2/3 of the operand loads of 256x128 tiles and 3/4 of their fragment reads
    // (4096^3: 145 -> 148 TFLOP/s; config 3: 137 -> 142; config 5's dX, (K, K) with K = 16384,
    // on them instead of 32-deep 128x128 slices).
    if (t.kernel == KERN_PIPE && splits == 1 && a_mode == LOAD_K && b_mode != LOAD_S &&
        mm % PIPE_TALL_M == 0 && nn % PIPE_WIDE_N == 0 && k % (PIPE_STAGES * 16) == 0 &&
        (t.tile == PIPE_TALL_M || (t.tile == GEMM_BM && t.slice_k == 32)) &&
        static_cast<uint64_t>(mm / PIPE_TALL_M) * (nn / PIPE_WIDE_N) * batch >= GEMM_CUS) {
        t.tile = PIPE_TALL_M;
        t.tile_n = PIPE_WIDE_N;
        t.tiles_m = mm / PIPE_TALL_M;
        t.tiles_n = nn / PIPE_WIDE_N;
        t.slice_k = 16;
        info.tile_m = PIPE_TALL_M;
        info.tile_n = PIPE_WIDE_N;
    }
    // Stream-K: full 128x128 tiles, at least one per compute unit, that the grids above would
    // spread unevenly (the busiest compute unit more than 10/9 of the mean: the rank-4 48^6
    // product, 2304^3, has 324 tiles for 256 compute units) take gemm_f32_sk, which gives each
    // compute unit an equal run of pipeline steps over 32-deep slices.
    if (splits == 1 && a_mode != LOAD_S && b_mode != LOAD_S && mm % GEMM_BM == 0 && nn % GEMM_BN == 0 &&
        k % (PIPE_STAGES * 32) == 0) {
        const uint64_t t128 = static_cast<uint64_t>(mm / GEMM_BM) * (nn / GEMM_BN) * batch;
        const uint64_t rounds = (t128 + SK_RANGES - 1) / SK_RANGES;
        if (t128 >= SK_RANGES && 10 * t128 < 9 * rounds * SK_RANGES) {
            t.kernel = KERN_SK;
            t.tile = t.tile_n = GEMM_BM;
            t.tiles_m = mm / GEMM_BM;
            t.tiles_n = nn / GEMM_BN;
            t.slice_k = 32;
            t.kgroups = 1;
            info.tile_m = info.tile_n = GEMM_BM;
        }
    }
    info.kgroups = t.kgroups;
    info.kernel = t.kernel == KERN_SK       ? LG_KERNEL_STREAMK
                  : t.kernel == KERN_TILE   ? LG_KERNEL_TILE
                  : t.kernel == KERN_PIPE   ? LG_KERNEL_PIPELINED
                  : t.kernel == KERN_DIRECT ? LG_KERNEL_DIRECT
                  : t.kernel == KERN_SMALL  ? LG_KERNEL_SMALL
                                            : LG_KERNEL_WAVE;
    t.splits = splits;
    t.k_chunk = chunk;
    info.splits = splits;
    info.k_chunk = chunk;
    info.workgroups = gemm_workgroups(t);
    if (t.kernel == KERN_SK) info.scratch_bytes = SK_PARTIAL_BYTES;
    if (splits == 1) {
        info.kind = LG_PLAN_TILED;
        return p;
    }
    info.kind = LG_PLAN_SPLIT;
    info.scratch_bytes = static_cast<uint64_t>(splits) * split_bytes;
    ReduceArgs& r = p.reduce;
    r.c = cptr;
    r.c_sb = t.c_sb;
    r.c_sm = t.c_sm;
    r.c_sn = t.c_sn;
    r.m = mm;
    r.n = nn;
    r.batch = batch;
    r.splits = splits;
    r.beta = beta;
    r.slices = useful < 65536 && splits >= 64 ? 16 : 4;
    return p;
}

void prepare_views(const View& a, const View& b, const View& c, bool half) {
    const uint32_t esz = half ? 2 : 4;
    validate(a, esz);
    validate(b, esz);
    validate(c, esz);
}

Plan plan_contract(float alpha, const lg_view* a_c, const char* la, const lg_view* b_c,
                   const char* lb, float beta, const lg_view* c_c, const char* lc, View* a,
                   View* b, View* c, bool half = false) {
    *a = view_from_c(a_c, "A");
    *b = view_from_c(b_c, "B");
    *c = view_from_c(c_c, "C");
    prepare_views(*a, *b, *c, half);
    const std::string sa = parse_labels(la, a->rank(), "A");
    const std::string sb = parse_labels(lb, b->rank(), "B");
    const std::string sc = parse_labels(lc, c->rank(), "C");
    return plan_merged(*a, *b, *c, merge_all(groups_from_labels(*a, sa, *b, sb, *c, sc)), alpha,
                       beta, half);
}

Plan plan_gemm(float alpha, const lg_view* a_c, const lg_view* b_c, float beta, const lg_view* c_c,
               View* a, View* b, View* c, bool half = false) {
    *a = view_from_c(a_c, "A");
    *b = view_from_c(b_c, "B");
    *c = view_from_c(c_c, "C");
    prepare_views(*a, *b, *c, half);
    return plan_merged(*a, *b, *c, merge_all(groups_from_gemm(*a, *b, *c)), alpha, beta, half);
}

// Plans of the last few gemm calls on this thread, keyed on every input the planner reads: the
// three views' fields, alpha and beta as bits and the element width. A call repeating one of
// them (the same views again, as a training loop or a benchmark makes) skips the planner's
// work, about 1 us of host time against a few us per launch; a plan is a function of exactly
// these inputs, so a hit returns what planning would. Inputs the planner rejects are never
// stored, so they are rejected again.
struct CachedPlan {
    bool used = false;
    bool half = false;
    uint32_t alpha_bits = 0, beta_bits = 0;
    lg_view v[3];
    Plan plan;
};
constexpr int PLAN_CACHE = 4;
thread_local CachedPlan plan_cache[PLAN_CACHE];
thread_local int plan_cache_next = 0;

bool cacheable(const lg_view* v) {
    return v != nullptr && v->rank <= LG_MAX_RANK && v->nstrides <= LG_MAX_RANK;
}
bool same_view(const lg_view& x, const lg_view* y) {
    if (x.base != y->base || x.bytes != y->bytes || x.offset != y->offset || x.rank != y->rank ||
        x.nstrides != y->nstrides) {
        return false;
    }
    for (uint32_t i = 0; i < x.rank; ++i) {
        if (x.shape[i] != y->shape[i]) return false;
    }
    for (uint32_t i = 0; i < x.nstrides; ++i) {
        if (x.strides[i] != y->strides[i]) return false;
    }
    return true;
}

Plan plan_gemm_cached(float alpha, const lg_view* a, const lg_view* b, float beta, const lg_view* c,
                      bool half = false) {
    View va, vb, vc;
    if (!cacheable(a) || !cacheable(b) || !cacheable(c)) return plan_gemm(alpha, a, b, beta, c, &va, &vb, &vc, half);
    uint32_t ab, bb;
    std::memcpy(&ab, &alpha, 4);
    std::memcpy(&bb, &beta, 4);
    for (const CachedPlan& e : plan_cache) {
        if (e.used && e.half == half && e.alpha_bits == ab && e.beta_bits == bb && same_view(e.v[0], a) &&
            same_view(e.v[1], b) && same_view(e.v[2], c)) {
            return e.plan;
        }
    }
    Plan p = plan_gemm(alpha, a, b, beta, c, &va, &vb, &vc, half);
    CachedPlan& e = plan_cache[plan_cache_next];
    plan_cache_next = (plan_cache_next + 1) % PLAN_CACHE;
    e.used = true;
    e.half = half;
    e.alpha_bits = ab;
    e.beta_bits = bb;
    e.v[0] = *a;
    e.v[1] = *b;
    e.v[2] = *c;
    e.plan = p;
    return p;
}

// Device scratch handed to a split or split-dot plan's launches: the partials.
struct Scratch {
    float* partial = nullptr;
    uint32_t* counters = nullptr;  // stream-K tickets, SK_COUNTER_BYTES after the partials
};

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    check_hip(hipStreamIsCapturing(s, &st), "hipStreamIsCapturing");
    return st != hipStreamCaptureStatusNone;
}

bool needs_scratch(const Plan& p) {
    return !p.half && (p.info.kind == LG_PLAN_SPLIT || (p.info.kind == LG_PLAN_DOT && p.dot.splits > 1) ||
                       (p.info.kind == LG_PLAN_TILED && p.gemm.kernel == KERN_SK));
}

Scratch scratch_at(void* base) {
    Scratch sc;
    sc.partial = static_cast<float*>(base);
    sc.counters = reinterpret_cast<uint32_t*>(static_cast<char*>(base) + SPLIT_PARTIAL_MAX);
    return sc;
}

// Enqueues the plan's launches; split and split-dot plans use `sc`.
void launch_plan(lg_ctx* ctx, hipStream_t s, Plan& p, const Scratch& sc) {
    if (p.half) {
        switch (p.info.kind) {
            case LG_PLAN_ZERO:
            case LG_PLAN_SCALE:
                launch_fill_half(ctx, s, p.hfill);
                return;
            case LG_PLAN_GENERAL:
                launch_general_half(ctx, s, p.hgeneral);
                return;
            case LG_PLAN_TILED:
                launch_gemm_half(ctx, s, p.hgemm, static_cast<int>(p.info.a_mode),
                                 static_cast<int>(p.info.b_mode));
                return;
            default:
                return;  // empty
        }
    }
    switch (p.info.kind) {
        case LG_PLAN_EMPTY:
            return;
        case LG_PLAN_ZERO:
        case LG_PLAN_SCALE:
            launch_fill(ctx, s, p.fill);
            return;
        case LG_PLAN_GENERAL:
            launch_general(ctx, s, p.general);
            return;
        case LG_PLAN_TILED:
            if (p.gemm.kernel == KERN_SK) {
                p.gemm.partial = sc.partial;
                p.gemm.counters = sc.counters;
            }
            launch_gemm(ctx, s, p.gemm, static_cast<int>(p.info.a_mode),
                        static_cast<int>(p.info.b_mode));
            return;
        case LG_PLAN_SPLIT:
            p.gemm.partial = sc.partial;
            p.reduce.partial = sc.partial;
            launch_gemm(ctx, s, p.gemm, static_cast<int>(p.info.a_mode),
                        static_cast<int>(p.info.b_mode));
            launch_reduce(ctx, s, p.reduce);
            return;
        case LG_PLAN_DOT:
            p.dot.partial = sc.partial;
            launch_dot(ctx, s, p.dot, p.info.a_mode == LG_LOAD_K_CONTIG);
            return;
    }
}

void execute(lg_ctx* ctx, hipStream_t s, Plan& p) {
    if (!needs_scratch(p)) {
        launch_plan(ctx, s, p, Scratch{});
        return;
    }
    // The context's scratch, made with the context and never grown, so this path allocates
    // nothing and never blocks. Eager calls are ordered after the previous user: calls on the
    // context's own stream by the stream, any other pair by split_event (also when both are
    // one caller's stream handle: the handle may name a new stream created after the old one
    // was destroyed with work still queued). A call under stream capture cannot wait on or
    // record an eager event; it is ordered only by its own stream, so replays of the graph
    // must not overlap the context's other split work (the caller orders them).
    std::lock_guard<std::mutex> hold(ctx->split_lock);
    const bool cap = capturing(s);
    if (!cap) {
        const bool own = s == ctx->stream && ctx->split_stream == ctx->stream;
        if (ctx->split_stream != nullptr && !own) {
            if (ctx->split_stream == ctx->stream) {
                check_hip(hipEventRecord(ctx->split_event, ctx->stream), "hipEventRecord");
            }
            check_hip(hipStreamWaitEvent(s, ctx->split_event, 0), "hipStreamWaitEvent");
        }
    }
    launch_plan(ctx, s, p, scratch_at(ctx->split_scratch));
    if (!cap) {
        ctx->split_stream = s;
        if (s != ctx->stream) {
            // Marks the end of this use for a later call on another stream; the context's own
            // stream outlives the buffer, so its uses are marked only when needed.
            check_hip(hipEventRecord(ctx->split_event, s), "hipEventRecord");
        }
    }
}

void run(lg_ctx* ctx, void* stream, Plan plan, bool wait) {
    set_device(ctx);
    hipStream_t s = pick_stream(ctx, stream);
    execute(ctx, s, plan);
    if (wait) check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
}

}  // namespace

void enqueue_gemm_fixed_scratch(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                                const lg_view* b, float beta, const lg_view* c,
                                uint64_t partial_cap, float* (*scratch)(lg_ctx*)) {
    View va, vb, vc;
    Plan plan = plan_gemm(alpha, a, b, beta, c, &va, &vb, &vc);
    if (plan.info.scratch_bytes > partial_cap) {
        fail_invalid("product needs " + std::to_string(plan.info.scratch_bytes) +
                     " bytes of split scratch; at most " + std::to_string(partial_cap) +
                     " are available");
    }
    set_device(ctx);
    hipStream_t s = pick_stream(ctx, stream);
    launch_plan(ctx, s, plan, needs_scratch(plan) ? scratch_at(scratch(ctx)) : Scratch{});
}

void enqueue_gemm_views(lg_ctx* ctx, hipStream_t s, float alpha, const View& a, const View& b,
                        float beta, const View& c) {
    Plan plan = plan_merged(a, b, c, merge_all(groups_from_gemm(a, b, c)), alpha, beta, false);
    set_device(ctx);
    execute(ctx, s, plan);
}

}  // namespace lg

using namespace lg;

extern "C" {

lg_status lg_encode_contract_f32(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                                 const char* a_labels, const lg_view* b, const char* b_labels,
                                 float beta, const lg_view* c, const char* c_labels) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        View va, vb, vc;
        run(ctx, stream,
            plan_contract(alpha, a, a_labels, b, b_labels, beta, c, c_labels, &va, &vb, &vc), false);
    });
}

lg_status lg_contract_f32(lg_ctx* ctx, float alpha, const lg_view* a, const char* a_labels,
                          const lg_view* b, const char* b_labels, float beta, const lg_view* c,
                          const char* c_labels) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        View va, vb, vc;
        run(ctx, nullptr,
            plan_contract(alpha, a, a_labels, b, b_labels, beta, c, c_labels, &va, &vb, &vc), true);
    });
}

lg_status lg_encode_gemm_f32(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                             const lg_view* b, float beta, const lg_view* c) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        run(ctx, stream, plan_gemm_cached(alpha, a, b, beta, c), false);
    });
}

lg_status lg_gemm_f32(lg_ctx* ctx, float alpha, const lg_view* a, const lg_view* b, float beta,
                      const lg_view* c) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        run(ctx, nullptr, plan_gemm_cached(alpha, a, b, beta, c), true);
    });
}

lg_status lg_gemm_nowait_f32(lg_ctx* ctx, float alpha, const lg_view* a, const lg_view* b,
                             float beta, const lg_view* c) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        run(ctx, nullptr, plan_gemm_cached(alpha, a, b, beta, c), false);
    });
}

lg_status lg_plan_contract_f32(float alpha, const lg_view* a, const char* a_labels,
                               const lg_view* b, const char* b_labels, float beta,
                               const lg_view* c, const char* c_labels, lg_contract_plan* out) {
    return guarded([&] {
        if (out == nullptr) fail_invalid("null output plan");
        View va, vb, vc;
        *out = plan_contract(alpha, a, a_labels, b, b_labels, beta, c, c_labels, &va, &vb, &vc).info;
    });
}

lg_status lg_plan_gemm_f32(float alpha, const lg_view* a, const lg_view* b, float beta,
                           const lg_view* c, lg_contract_plan* out) {
    return guarded([&] {
        if (out == nullptr) fail_invalid("null output plan");
        View va, vb, vc;
        *out = plan_gemm(alpha, a, b, beta, c, &va, &vb, &vc).info;
    });
}

lg_status lg_encode_contract_f16(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                                 const char* a_labels, const lg_view* b, const char* b_labels,
                                 float beta, const lg_view* c, const char* c_labels) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        View va, vb, vc;
        run(ctx, stream,
            plan_contract(alpha, a, a_labels, b, b_labels, beta, c, c_labels, &va, &vb, &vc, true), false);
    });
}

lg_status lg_contract_f16(lg_ctx* ctx, float alpha, const lg_view* a, const char* a_labels,
                          const lg_view* b, const char* b_labels, float beta, const lg_view* c,
                          const char* c_labels) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        View va, vb, vc;
        run(ctx, nullptr,
            plan_contract(alpha, a, a_labels, b, b_labels, beta, c, c_labels, &va, &vb, &vc, true), true);
    });
}

lg_status lg_encode_gemm_f16(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                             const lg_view* b, float beta, const lg_view* c) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        View va, vb, vc;
        run(ctx, stream, plan_gemm(alpha, a, b, beta, c, &va, &vb, &vc, true), false);
    });
}

lg_status lg_gemm_f16(lg_ctx* ctx, float alpha, const lg_view* a, const lg_view* b, float beta,
                      const lg_view* c) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        View va, vb, vc;
        run(ctx, nullptr, plan_gemm(alpha, a, b, beta, c, &va, &vb, &vc, true), true);
    });
}

lg_status lg_gemm_nowait_f16(lg_ctx* ctx, float alpha, const lg_view* a, const lg_view* b,
                             float beta, const lg_view* c) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        View va, vb, vc;
        run(ctx, nullptr, plan_gemm(alpha, a, b, beta, c, &va, &vb, &vc, true), false);
    });
}

lg_status lg_plan_contract_f16(float alpha, const lg_view* a, const char* a_labels,
                               const lg_view* b, const char* b_labels, float beta,
                               const lg_view* c, const char* c_labels, lg_contract_plan* out) {
    return guarded([&] {
        if (out == nullptr) fail_invalid("null output plan");
        View va, vb, vc;
        *out = plan_contract(alpha, a, a_labels, b, b_labels, beta, c, c_labels, &va, &vb, &vc, true).info;
    });
}

lg_status lg_plan_gemm_f16(float alpha, const lg_view* a, const lg_view* b, float beta,
                           const lg_view* c, lg_contract_plan* out) {
    return guarded([&] {
        if (out == nullptr) fail_invalid("null output plan");
        View va, vb, vc;
        *out = plan_gemm(alpha, a, b, beta, c, &va, &vb, &vc, true).info;
    });
}

}  // extern "C"
