// CPU ASTC LDR encoder behind akv_encode. The reference encodes with Arm
// astcenc 5.7.0 (astc_kv/bridge.cpp:18-26), which is not available here; this
// is an encoder of our own. Any block it emits is a valid ASTC LDR block, so
// decode parity (the property the read path depends on) is independent of
// the encoder's search choices.
//
// Search per block:
//   * constant blocks -> LDR void-extent block;
//   * colour endpoint mode from the channel structure: luminance (CEM 0),
//     luminance+alpha (CEM 4), RGB (CEM 8) or RGBA (CEM 12);
//   * 1 partition, plus 2 and 3 (4 at quality >= 90) partitions whose seeds
//     are chosen by matching the partition table against a k-means clustering
//     of the texels (the best 1, 2 or 4 seeds per count, more at higher
//     quality);
//   * weight grids: the full footprint and, at high effort, grids one or two
//     texels smaller; every weight range whose colour data still fits;
//   * per candidate: principal-axis line fit, up to four rounds of
//     least-squares endpoint refinement, then the candidate is packed and
//     decoded exactly and scored by squared error of the decoded FP16 texels;
//   * at quality >= 90, luminance candidates on the full grid also try the
//     neighbouring quantised endpoint codes (3 x 3 per partition, in value
//     order) and keep the pair of least error.
#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "astc_bits.h"
#include "astc_codec.h"

namespace akv {

namespace {

struct GridMode {
    uint32_t bits;   // block mode field
    int gw, gh, range, wbits;
    bool identity;
};

struct Plan {
    const AkvTables* t = nullptr;
    std::vector<GridMode> modes;          // single-plane modes, one per (grid, range)
    uint8_t nearest_color[kNumRanges][256];
    // The codes of the next lower and next higher colour value of a range
    // (the code itself at either end).
    uint8_t color_down[kNumRanges][256], color_up[kNumRanges][256];
    uint8_t nearest_weight[12][65];
    uint16_t trit_code[243];
    uint8_t quint_code[125];
    // Infill taps of each texel for each grid size: (grid index, factor/16).
    struct Tap {
        uint8_t idx[4];
        uint8_t f[4];
    };
    struct Gather {
        std::vector<std::pair<uint8_t, uint8_t>> from;  // (texel, factor) per grid point
    };
    // Texel membership masks of each partition for 2/3/4 partitions and seed.
    uint64_t part_mask[3][1024][4];
    std::map<int, std::vector<Tap>> taps;       // key gw*16+gh: infill taps per texel
    std::map<int, std::vector<Gather>> gather;  // key gw*16+gh: transpose, per grid point
};

const Plan& plan_for(const AkvTables& t) {
    static std::mutex mu;
    static std::map<const AkvTables*, std::unique_ptr<Plan>> plans;
    std::lock_guard<std::mutex> lock(mu);
    auto it = plans.find(&t);
    if (it != plans.end()) return *it->second;
    auto p = std::make_unique<Plan>();
    p->t = &t;
    const int bx = int(t.block_x), by = int(t.block_y);
    std::map<int, bool> seen;
    for (uint32_t m = 0; m < 2048; ++m) {
        uint32_t md = t.block_mode[m];
        if (!md || mode_dual(md)) continue;
        int key = int(mode_gw(md)) * 256 + int(mode_gh(md)) * 16 + int(mode_range(md));
        if (seen.count(key)) continue;
        seen[key] = true;
        p->modes.push_back({m, int(mode_gw(md)), int(mode_gh(md)), int(mode_range(md)), int(mode_wbits(md)),
                            mode_identity(md) != 0});
    }
    for (int r = 0; r < kNumRanges; ++r) {
        int levels = ise_levels(r);
        for (int target = 0; target < 256; ++target) {
            int best = 0, bestd = 1 << 30;
            for (int v = 0; v < levels; ++v) {
                int d = std::abs(int(t.color_unq[r][v]) - target);
                if (d < bestd) { bestd = d; best = v; }
            }
            p->nearest_color[r][target] = uint8_t(best);
        }
        for (int v = 0; v < levels; ++v) {
            const int u = t.color_unq[r][v];
            int dn = v, up = v, dnu = -1, upu = 256;
            for (int c = 0; c < levels; ++c) {
                const int cu = t.color_unq[r][c];
                if (cu < u && cu > dnu) { dnu = cu; dn = c; }
                if (cu > u && cu < upu) { upu = cu; up = c; }
            }
            p->color_down[r][v] = uint8_t(dn);
            p->color_up[r][v] = uint8_t(up);
        }
    }
    for (int r = 0; r < 12; ++r) {
        int levels = ise_levels(r);
        for (int target = 0; target <= 64; ++target) {
            int best = 0, bestd = 1 << 30;
            for (int v = 0; v < levels; ++v) {
                int d = std::abs(int(t.weight_unq[r][v]) - target);
                if (d < bestd) { bestd = d; best = v; }
            }
            p->nearest_weight[r][target] = uint8_t(best);
        }
    }
    // Inverse trit/quint block tables; the smallest code is kept, which also has
    // zero bits wherever a truncated last group omits its tail.
    std::fill(p->trit_code, p->trit_code + 243, 0xFFFF);
    for (int T = 255; T >= 0; --T) {
        unsigned d = t.trit[T];
        int idx = 0;
        for (int j = 4; j >= 0; --j) idx = idx * 3 + int((d >> (2 * j)) & 3);
        p->trit_code[idx] = uint16_t(T);
    }
    for (int Q = 127; Q >= 0; --Q) {
        unsigned d = t.quint[Q];
        int idx = int(d & 7) + 5 * int((d >> 3) & 7) + 25 * int((d >> 6) & 7);
        p->quint_code[idx] = uint8_t(Q);
    }
    std::memset(p->part_mask, 0, sizeof(p->part_mask));
    for (int k = 0; k < 3; ++k)
        for (int seed = 0; seed < 1024; ++seed)
            for (int i = 0; i < bx * by; ++i)
                p->part_mask[k][seed][(t.partition[k][seed][i >> 4] >> (2 * (i & 15))) & 3] |= uint64_t(1) << i;
    for (const GridMode& g : p->modes) {
        int key = g.gw * 16 + g.gh;
        if (p->taps.count(key)) continue;
        std::vector<Plan::Tap> taps(bx * by);
        const int ds = (1024 + bx / 2) / (bx - 1), dt = (1024 + by / 2) / (by - 1);
        for (int y = 0; y < by; ++y)
            for (int x = 0; x < bx; ++x) {
                int gs = (ds * x * (g.gw - 1) + 32) >> 6, gt = (dt * y * (g.gh - 1) + 32) >> 6;
                int fs = gs & 15, ft = gt & 15, base = (gs >> 4) + (gt >> 4) * g.gw;
                int f11 = (fs * ft + 8) >> 4;
                Plan::Tap& tp = taps[y * bx + x];
                int idx[4] = {base, base + 1, base + g.gw, base + g.gw + 1};
                int f[4] = {16 - fs - ft + f11, fs - f11, ft - f11, f11};
                for (int k = 0; k < 4; ++k) {
                    tp.f[k] = uint8_t(f[k]);
                    tp.idx[k] = uint8_t(f[k] ? idx[k] : base);
                }
            }
        std::vector<Plan::Gather> gather(g.gw * g.gh);
        for (int i = 0; i < bx * by; ++i)
            for (int k = 0; k < 4; ++k)
                if (taps[i].f[k]) gather[taps[i].idx[k]].from.push_back({uint8_t(i), taps[i].f[k]});
        p->taps[key] = std::move(taps);
        p->gather[key] = std::move(gather);
    }
    const Plan& ref = *p;
    plans.emplace(&t, std::move(p));
    return ref;
}

void ise_pack(const Plan& plan, const int* values, int count, int range, Bits128& dst, int start) {
    const int n = ise_bits(range);
    int pos = start;
    if (ise_trit(range)) {
        static const int tbits[5] = {2, 2, 1, 2, 1}, tshift[5] = {0, 2, 4, 5, 7};
        for (int i = 0; i < count; i += 5) {
            int idx = 0;
            for (int j = 4; j >= 0; --j) idx = idx * 3 + (i + j < count ? values[i + j] >> n : 0);
            unsigned T = plan.trit_code[idx];
            for (int j = 0; j < 5 && i + j < count; ++j) {
                dst.put(pos, n, uint64_t(values[i + j] & ((1 << n) - 1)));
                pos += n;
                dst.put(pos, tbits[j], (T >> tshift[j]) & ((1u << tbits[j]) - 1));
                pos += tbits[j];
            }
        }
    } else if (ise_quint(range)) {
        static const int qbits[3] = {3, 2, 2}, qshift[3] = {0, 3, 5};
        for (int i = 0; i < count; i += 3) {
            int idx = 0;
            for (int j = 2; j >= 0; --j) idx = idx * 5 + (i + j < count ? values[i + j] >> n : 0);
            unsigned Q = plan.quint_code[idx];
            for (int j = 0; j < 3 && i + j < count; ++j) {
                dst.put(pos, n, uint64_t(values[i + j] & ((1 << n) - 1)));
                pos += n;
                dst.put(pos, qbits[j], (Q >> qshift[j]) & ((1u << qbits[j]) - 1));
                pos += qbits[j];
            }
        }
    } else {
        for (int i = 0; i < count; ++i, pos += n) dst.put(pos, n, uint64_t(values[i]));
    }
}

inline float fp16_value(uint16_t h) {
    int e = (h >> 10) & 31, m = h & 0x3FF;
    if (e == 0) return float(m) * (1.0f / 16777216.0f);
    return std::ldexp(1.0f + float(m) / 1024.0f, e - 15);
}

struct BlockInput {
    int ntex = 0;
    int nch = 0;           // active channels
    int ch[4] = {0, 0, 0, 0};
    int cem = 0;
    float x[kMaxTexels][4];  // active channels only
    float full[kMaxTexels][4];
};

// Colour values (ISE order) for one partition's endpoints, given 8-bit targets.
int cem_values(int cem, const int* lo, const int* hi, int* out) {
    switch (cem) {
        case 0: out[0] = lo[0]; out[1] = hi[0]; return 2;
        case 4: out[0] = lo[0]; out[1] = hi[0]; out[2] = lo[3]; out[3] = hi[3]; return 4;
        case 8: for (int c = 0; c < 3; ++c) { out[2 * c] = lo[c]; out[2 * c + 1] = hi[c]; } return 6;
        default: for (int c = 0; c < 4; ++c) { out[2 * c] = lo[c]; out[2 * c + 1] = hi[c]; } return 8;
    }
}

struct Candidate {
    uint8_t block[16];
    double err = 1e30;
};

// Score a packed block by decoding it exactly.
double block_error(const AkvTables& t, const BlockInput& in, const uint8_t* block) {
    uint16_t dec[kMaxTexels * 4];
    decode_block_fp16(t, block, dec);
    double e = 0;
    for (int i = 0; i < in.ntex; ++i)
        for (int k = 0; k < in.nch; ++k) {
            double d = double(fp16_value(dec[4 * i + in.ch[k]])) - in.x[i][k];
            e += d * d;
        }
    return e;
}

void void_extent(const BlockInput& in, uint8_t* out) {
    Bits128 b;
    b.put(0, 12, 0xDFC);                 // void-extent selector, LDR, reserved bits set
    b.put(12, 52, ~uint64_t(0));         // unbounded extent
    for (int c = 0; c < 4; ++c) {
        // The decoder truncates c/65536 to FP16; pick the UNORM16 value whose
        // FP16 image is nearest v among the FP16 neighbours of v.
        double v = std::clamp(double(in.full[0][c]), 0.0, 1.0);
        uint32_t best = 0;
        double bestd = 1e30;
        uint32_t guess = uint32_t(std::min(v * 65536.0, 65535.0));
        uint32_t cands[4] = {guess, 65535u, 0u, 0u};
        uint16_t hb = unorm16_to_fp16_bits(guess);
        double below = double(fp16_value(hb));
        double above = double(fp16_value(uint16_t(hb + 1)));
        cands[2] = uint32_t(std::min(above * 65536.0, 65535.0));
        cands[3] = uint32_t(below * 65536.0);
        for (uint32_t cand : cands) {
            double d = std::fabs(double(fp16_value(unorm16_to_fp16_bits(cand))) - v);
            if (d < bestd) { bestd = d; best = cand; }
        }
        b.put(64 + 16 * c, 16, best);
    }
    b.store(out);
}

// Endpoints (in active-channel space, [0,1]) of one partition's texels: mean plus
// the extent of the projections on the principal axis.
struct Members {
    uint8_t idx[kMaxTexels];
    int n = 0;
    void push(int i) { idx[n++] = uint8_t(i); }
    const uint8_t* begin() const { return idx; }
    const uint8_t* end() const { return idx + n; }
    bool empty() const { return n == 0; }
    size_t size() const { return size_t(n); }
};

void line_fit(const BlockInput& in, const Members& idx, float* lo, float* hi) {
    const int C = in.nch;
    float mean[4] = {0, 0, 0, 0};
    if (idx.empty()) {
        for (int k = 0; k < C; ++k) lo[k] = hi[k] = 0;
        return;
    }
    for (int i : idx)
        for (int k = 0; k < C; ++k) mean[k] += in.x[i][k];
    for (int k = 0; k < C; ++k) mean[k] /= float(idx.size());
    float cov[4][4] = {};
    for (int i : idx)
        for (int a = 0; a < C; ++a)
            for (int b = 0; b < C; ++b) cov[a][b] += (in.x[i][a] - mean[a]) * (in.x[i][b] - mean[b]);
    float dir[4] = {1, 1, 1, 1};
    for (int it = 0; it < 10; ++it) {
        float nd[4] = {0, 0, 0, 0}, norm = 0;
        for (int a = 0; a < C; ++a) {
            for (int b = 0; b < C; ++b) nd[a] += cov[a][b] * dir[b];
            norm += nd[a] * nd[a];
        }
        if (norm < 1e-30f) break;
        norm = 1.0f / std::sqrt(norm);
        for (int a = 0; a < C; ++a) dir[a] = nd[a] * norm;
    }
    float tmin = 1e30f, tmax = -1e30f;
    for (int i : idx) {
        float p = 0;
        for (int k = 0; k < C; ++k) p += (in.x[i][k] - mean[k]) * dir[k];
        tmin = std::min(tmin, p);
        tmax = std::max(tmax, p);
    }
    for (int k = 0; k < C; ++k) {
        lo[k] = std::clamp(mean[k] + tmin * dir[k], 0.0f, 1.0f);
        hi[k] = std::clamp(mean[k] + tmax * dir[k], 0.0f, 1.0f);
    }
}

struct PartitionLayout {
    int count = 1;
    int seed = 0;
    uint8_t of[kMaxTexels] = {};
};

// Build one packed candidate for a partition layout, grid mode and effort.
void make_candidate(const Plan& plan, const BlockInput& in, const PartitionLayout& pl, const GridMode& gm,
                    int refine, Candidate& best, bool polish = false) {
    const AkvTables& t = *plan.t;
    const int pc = pl.count, cem = in.cem;
    const int pairs = pc * ((cem >> 2) + 1);
    if (2 * pairs > 18) return;
    const int config = pc == 1 ? 17 : 29;
    const int avail = 128 - gm.wbits - config;
    if (avail <= 0) return;
    const int crange = t.color_range[pairs][std::min(avail, 127)];
    if (crange < kRange6) return;
    const int C = in.nch;
    Members members[4];
    for (int i = 0; i < in.ntex; ++i) members[pl.of[i]].push(i);
    float lo[4][4], hi[4][4];
    for (int p = 0; p < pc; ++p) line_fit(in, members[p], lo[p], hi[p]);
    const auto& taps = plan.taps.at(gm.gw * 16 + gm.gh);
    const auto& gather = plan.gather.at(gm.gw * 16 + gm.gh);
    const int ngrid = gm.gw * gm.gh;
    int qlo[4][4], qhi[4][4];       // quantised ISE values per partition/active channel
    int elo[4][4], ehi[4][4];       // their 8-bit unquantised values
    int gridq[64];
    for (int pass = 0; pass <= refine; ++pass) {
        // Quantise endpoints.
        for (int p = 0; p < pc; ++p) {
            int s_lo = 0, s_hi = 0;
            for (int k = 0; k < C; ++k) {
                qlo[p][k] = plan.nearest_color[crange][int(std::lround(lo[p][k] * 255.0f))];
                qhi[p][k] = plan.nearest_color[crange][int(std::lround(hi[p][k] * 255.0f))];
                elo[p][k] = t.color_unq[crange][qlo[p][k]];
                ehi[p][k] = t.color_unq[crange][qhi[p][k]];
                if (k < 3) { s_lo += elo[p][k]; s_hi += ehi[p][k]; }
            }
            // RGB(A) direct modes swap and blue-contract when the second
            // endpoint sums lower; keep the stored order canonical instead.
            if ((cem == 8 || cem == 12) && s_hi < s_lo) {
                for (int k = 0; k < C; ++k) {
                    std::swap(qlo[p][k], qhi[p][k]);
                    std::swap(elo[p][k], ehi[p][k]);
                }
            }
        }
        // Ideal texel weights by projection on the quantised segment.
        float ideal[kMaxTexels];
        for (int i = 0; i < in.ntex; ++i) {
            int p = pl.of[i];
            float num = 0, den = 0;
            for (int k = 0; k < C; ++k) {
                float a = elo[p][k] / 255.0f, d = (ehi[p][k] - elo[p][k]) / 255.0f;
                num += (in.x[i][k] - a) * d;
                den += d * d;
            }
            ideal[i] = den > 0 ? std::clamp(num / den, 0.0f, 1.0f) * 64.0f : 0.0f;
        }
        // Down-sample to the grid with the transpose of the infill taps.
        for (int g = 0; g < ngrid; ++g) {
            float num = 0, den = 0;
            for (const auto& tf : gather[g].from) {
                num += tf.second * ideal[tf.first];
                den += tf.second;
            }
            float w = den > 0 ? num / den : 0.0f;
            gridq[g] = plan.nearest_weight[gm.range][std::clamp(int(std::lround(w)), 0, 64)];
        }
        if (pass == refine) break;
        // Least-squares endpoints for the decoded texel weights.
        float a_tex[kMaxTexels];
        for (int i = 0; i < in.ntex; ++i) {
            int acc = 0;
            for (int k = 0; k < 4; ++k) acc += taps[i].f[k] * t.weight_unq[gm.range][gridq[taps[i].idx[k]]];
            a_tex[i] = float((acc + 8) >> 4) / 64.0f;
        }
        for (int p = 0; p < pc; ++p) {
            double s00 = 0, s01 = 0, s11 = 0, r0[4] = {}, r1[4] = {};
            for (int i : members[p]) {
                double a = a_tex[i], b = 1.0 - a;
                s00 += b * b; s01 += a * b; s11 += a * a;
                for (int k = 0; k < C; ++k) { r0[k] += b * in.x[i][k]; r1[k] += a * in.x[i][k]; }
            }
            double det = s00 * s11 - s01 * s01;
            if (std::fabs(det) < 1e-9) continue;
            for (int k = 0; k < C; ++k) {
                lo[p][k] = float(std::clamp((r0[k] * s11 - r1[k] * s01) / det, 0.0, 1.0));
                hi[p][k] = float(std::clamp((r1[k] * s00 - r0[k] * s01) / det, 0.0, 1.0));
            }
        }
    }
    // Luminance, identity grid, highest effort: per partition, the quantised
    // endpoint pair and its neighbours one colour level down or up (nine
    // pairs), each with its texels' nearest weights; the pair of least
    // squared error (8-bit endpoint domain) stays.
    if (polish && C == 1 && gm.identity) {
        for (int p = 0; p < pc; ++p) {
            const int lo_c[3] = {qlo[p][0], plan.color_down[crange][qlo[p][0]], plan.color_up[crange][qlo[p][0]]};
            const int hi_c[3] = {qhi[p][0], plan.color_down[crange][qhi[p][0]], plan.color_up[crange][qhi[p][0]]};
            double best_e = 1e300;
            int bl = qlo[p][0], bh = qhi[p][0];
            for (int a = 0; a < 3; ++a)
                for (int c = 0; c < 3; ++c) {
                    const int el = t.color_unq[crange][lo_c[a]], eh = t.color_unq[crange][hi_c[c]];
                    double e = 0;
                    for (int i : members[p]) {
                        const float d = float(eh - el), x = in.x[i][0] * 255.0f - float(el);
                        const float w = d != 0.0f ? std::clamp(x / d, 0.0f, 1.0f) * 64.0f : 0.0f;
                        const int wq = t.weight_unq[gm.range][plan.nearest_weight[gm.range][std::clamp(int(std::lround(w)), 0, 64)]];
                        const double v = (el * (64 - wq) + eh * wq) / 64.0 - in.x[i][0] * 255.0;
                        e += v * v;
                    }
                    if (e < best_e) { best_e = e; bl = lo_c[a]; bh = hi_c[c]; }
                }
            qlo[p][0] = bl;
            qhi[p][0] = bh;
            elo[p][0] = t.color_unq[crange][bl];
            ehi[p][0] = t.color_unq[crange][bh];
            for (int i : members[p]) {
                const float d = float(ehi[p][0] - elo[p][0]), x = in.x[i][0] * 255.0f - float(elo[p][0]);
                const float w = d != 0.0f ? std::clamp(x / d, 0.0f, 1.0f) * 64.0f : 0.0f;
                gridq[i] = plan.nearest_weight[gm.range][std::clamp(int(std::lround(w)), 0, 64)];
            }
        }
    }
    // Pack.
    Bits128 b;
    b.put(0, 11, gm.bits);
    b.put(11, 2, uint64_t(pc - 1));
    if (pc == 1) {
        b.put(13, 4, uint64_t(cem));
    } else {
        b.put(13, 10, uint64_t(pl.seed));
        b.put(23, 6, uint64_t(cem) << 2);
    }
    int vals[18], nv = 0;
    for (int p = 0; p < pc; ++p) {
        int l[4] = {0, 0, 0, 0}, h[4] = {0, 0, 0, 0};
        if (cem == 0) { l[0] = qlo[p][0]; h[0] = qhi[p][0]; }
        else if (cem == 4) { l[0] = qlo[p][0]; h[0] = qhi[p][0]; l[3] = qlo[p][1]; h[3] = qhi[p][1]; }
        else for (int k = 0; k < C; ++k) { l[k] = qlo[p][k]; h[k] = qhi[p][k]; }
        nv += cem_values(cem, l, h, vals + nv);
    }
    ise_pack(plan, vals, nv, crange, b, config);
    Bits128 w;
    ise_pack(plan, gridq, ngrid, gm.range, w, 0);
    Bits128 wr = w.reversed();
    b.lo |= wr.lo;
    b.hi |= wr.hi;
    Candidate c;
    b.store(c.block);
    c.err = block_error(t, in, c.block);
    if (c.err < best.err) best = c;
}

// k-means labels of the texels into k clusters (active channels).
void cluster(const BlockInput& in, int k, uint8_t* label) {
    float centre[4][4];
    // Seed with texels spread along the first channel sum.
    std::vector<std::pair<float, int>> order(in.ntex);
    for (int i = 0; i < in.ntex; ++i) {
        float s = 0;
        for (int c = 0; c < in.nch; ++c) s += in.x[i][c];
        order[i] = {s, i};
    }
    std::sort(order.begin(), order.end());
    for (int j = 0; j < k; ++j) {
        int pick = order[(2 * j + 1) * in.ntex / (2 * k)].second;
        for (int c = 0; c < in.nch; ++c) centre[j][c] = in.x[pick][c];
    }
    for (int it = 0; it < 6; ++it) {
        for (int i = 0; i < in.ntex; ++i) {
            float bd = 1e30f;
            for (int j = 0; j < k; ++j) {
                float d = 0;
                for (int c = 0; c < in.nch; ++c) d += (in.x[i][c] - centre[j][c]) * (in.x[i][c] - centre[j][c]);
                if (d < bd) { bd = d; label[i] = uint8_t(j); }
            }
        }
        float sum[4][4] = {};
        int cnt[4] = {};
        for (int i = 0; i < in.ntex; ++i) {
            cnt[label[i]]++;
            for (int c = 0; c < in.nch; ++c) sum[label[i]][c] += in.x[i][c];
        }
        for (int j = 0; j < k; ++j)
            if (cnt[j])
                for (int c = 0; c < in.nch; ++c) centre[j][c] = sum[j][c] / float(cnt[j]);
    }
}

// Seeds whose partition pattern best matches the clustering (fewest
// mismatched texels over all label permutations).
std::vector<int> best_seeds(const Plan& plan, const BlockInput& in, int k, int keep) {
    uint8_t label[kMaxTexels];
    cluster(in, k, label);
    uint64_t lmask[4] = {0, 0, 0, 0};
    for (int i = 0; i < in.ntex; ++i) lmask[label[i]] |= uint64_t(1) << i;
    static const int perms3[6][3] = {{0, 1, 2}, {0, 2, 1}, {1, 0, 2}, {1, 2, 0}, {2, 0, 1}, {2, 1, 0}};
    std::vector<std::pair<int, int>> score;
    score.reserve(1024);
    for (int seed = 0; seed < 1024; ++seed) {
        const uint64_t* pmask = plan.part_mask[k - 2][seed];
        bool empty = false;
        for (int j = 0; j < k; ++j) empty |= pmask[j] == 0;
        if (empty) continue;
        int bestm = 1 << 30;
        if (k == 2) {
            bestm = std::min(__builtin_popcountll(pmask[0] ^ lmask[0]), __builtin_popcountll(pmask[0] ^ lmask[1]));
        } else {
            for (auto& pm : perms3) {
                int m = 0;
                for (int j = 0; j < 3; ++j) m += __builtin_popcountll(pmask[j] ^ lmask[pm[j]]);
                bestm = std::min(bestm, m);
            }
        }
        score.push_back({bestm, seed});
    }
    size_t n = std::min<size_t>(size_t(keep), score.size());
    std::partial_sort(score.begin(), score.begin() + n, score.end());
    std::vector<int> seeds;
    for (size_t i = 0; i < n; ++i) seeds.push_back(score[i].second);
    return seeds;
}

}  // namespace

void encode_block(const AkvTables& t, const float* texels, const EncoderOptions& opt, uint8_t* out) {
    const Plan& plan = plan_for(t);
    BlockInput in;
    in.ntex = int(t.block_x * t.block_y);
    bool constant = true, lum = true, opaque = true;
    for (int i = 0; i < in.ntex; ++i) {
        for (int c = 0; c < 4; ++c) {
            float v = std::clamp(texels[4 * i + c], 0.0f, 1.0f);
            if (std::isnan(texels[4 * i + c])) v = 0.0f;
            in.full[i][c] = v;
            if (v != in.full[0][c]) constant = false;
        }
        if (in.full[i][0] != in.full[i][1] || in.full[i][0] != in.full[i][2]) lum = false;
        if (in.full[i][3] != 1.0f) opaque = false;
    }
    if (constant) {
        void_extent(in, out);
        return;
    }
    if (lum && opaque) { in.cem = 0; in.nch = 1; in.ch[0] = 0; }
    else if (lum) { in.cem = 4; in.nch = 2; in.ch[0] = 0; in.ch[1] = 3; }
    else if (opaque) { in.cem = 8; in.nch = 3; in.ch[0] = 0; in.ch[1] = 1; in.ch[2] = 2; }
    else { in.cem = 12; in.nch = 4; for (int c = 0; c < 4; ++c) in.ch[c] = c; }
    for (int i = 0; i < in.ntex; ++i)
        for (int k = 0; k < in.nch; ++k) in.x[i][k] = in.full[i][in.ch[k]];

    const float q = opt.quality;
    const int refine = q < 30 ? 0 : (q < 70 ? 1 : q < 90 ? 2 : 4);
    const int bx = int(t.block_x), by = int(t.block_y);
    Candidate best;
    // Identity grid, every weight range, for each partition layout tried.
    std::vector<PartitionLayout> layouts(1);
    if (q >= 30) {
        const int max_parts = q >= 90 ? 4 : q >= 70 ? 3 : 2;
        for (int k = 2; k <= max_parts; ++k) {
            if (k * 2 * ((in.cem >> 2) + 1) > 18) break;
            const int keep = q >= 90 ? (k == 2 ? 4 : 2) : (q >= 70 && k == 2) ? 2 : 1;
            for (int seed : best_seeds(plan, in, k, keep)) {
                PartitionLayout pl;
                pl.count = k;
                pl.seed = seed;
                for (int i = 0; i < in.ntex; ++i)
                    pl.of[i] = uint8_t((t.partition[k - 2][seed][i >> 4] >> (2 * (i & 15))) & 3);
                layouts.push_back(pl);
            }
        }
    }
    int best_layout = 0;
    for (size_t li = 0; li < layouts.size(); ++li) {
        double before = best.err;
        for (const GridMode& g : plan.modes)
            if (g.identity) make_candidate(plan, in, layouts[li], g, refine, best, q >= 90);
        if (best.err < before) best_layout = int(li);
    }
    // Smaller weight grids for the winning layout at high effort.
    if (q >= 70)
        for (const GridMode& g : plan.modes)
            if (!g.identity && g.gw >= bx - 2 && g.gh >= by - 2)
                make_candidate(plan, in, layouts[best_layout], g, refine, best);
    if (best.err >= 1e29) {
        // No mode fits (cannot happen for supported footprints): emit the
        // average colour as a void-extent block.
        for (int c = 0; c < 4; ++c) {
            float s = 0;
            for (int i = 0; i < in.ntex; ++i) s += in.full[i][c];
            in.full[0][c] = s / float(in.ntex);
        }
        void_extent(in, out);
        return;
    }
    std::memcpy(out, best.block, 16);
}

int encode_image(const AkvTables& t, const float* rgba, unsigned w, unsigned h, const EncoderOptions& opt,
                 uint8_t* out, size_t bytes) {
    const unsigned bx = t.block_x, by = t.block_y;
    const unsigned cols = (w + bx - 1) / bx, rows = (h + by - 1) / by;
    if (bytes < size_t(cols) * rows * 16) return 1;
    float tex[kMaxTexels * 4];
    for (unsigned r = 0; r < rows; ++r)
        for (unsigned c = 0; c < cols; ++c) {
            for (unsigned y = 0; y < by; ++y)
                for (unsigned x = 0; x < bx; ++x) {
                    unsigned sy = std::min(r * by + y, h - 1), sx = std::min(c * bx + x, w - 1);
                    std::memcpy(tex + 4 * (y * bx + x), rgba + (size_t(sy) * w + sx) * 4, 16);
                }
            encode_block(t, tex, opt, out + 16 * (size_t(r) * cols + c));
        }
    return 0;
}

}  // namespace akv
