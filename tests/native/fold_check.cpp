// Host check of the exact parallel f32 fold (turboqwenfare_amd/csrc/tqf_fold.h
// and the wavefront procedure of tqf_sample.hip's fold_chunks / fold_row /
// fold_chunk_terms), emulated lane by lane on the CPU: for every test row the
// folded value must equal the plain sequential f32 sum from -0, bit for bit,
// and the inverse-CDF walk must stop where the sequential walk stops.
//
// Rows: the sampler's own terms (exponentials of N(0, s^2) logits at several
// temperatures, token order, and the sorted probabilities), a row whose
// exponentials span the subnormal range, rows built to hit the rule's corner
// cases (exact ties at every parity, a term that alone jumps several binades,
// sums that land exactly on a binade's top, runs of equal terms), random bit
// patterns over the whole finite range, and short and ragged lengths.
//
// Negative controls: the same procedure with the tie check removed, and with
// the top check removed, must each disagree with the sequential sum on some
// row, so the check can see either slip.
//
// Usage: fold_check [seed]; prints "rows R mismatches M control_tie T
// control_top U" on its last line.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <random>
#include <vector>

#include "tqf_fold.h"

using namespace tqf;

namespace {

constexpr uint32_t kWave = 64, kChunk = 4 * kWave;  // a fold unit: 256 terms, 4 per lane
constexpr uint32_t kNoHit = 0xffffffffu;

bool g_skip_tie = false, g_skip_top = false;  // the negative controls

uint32_t bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
float from(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

struct Info {
    uint32_t meta_a, q_a, meta_b, q_b;
};

// fold_chunks: two candidate grids for the chunk's start (the binade of the
// float64 sum of the chunks before it, and its neighbour on the side the
// estimate leans to), the chunk's saturated count and tie flag on each, and
// its term flags.
Info chunk_info(const std::vector<uint32_t> &t, uint32_t c, double before) {
    const uint32_t eb = bits((float)before), ee = eb >> 23;
    uint32_t ga = ee > 1u ? ee : 1u, gb = (eb >> 22) & 1u ? ga + 1u : (ga > 1u ? ga - 1u : 2u);
    if (ee >= 254u) ga = gb = 255u;
    uint32_t qa = 0, qb = 0, flags = 0;
    bool ta = false, tb = false;
    for (uint32_t i = c * kChunk; i < (c + 1) * kChunk && i < t.size(); ++i) {
        const uint32_t fl = term_flags(t[i]);
        flags |= fl;
        bool tie_a, tie_b;
        const uint32_t ua = grid_units(from(t[i]), std::min(ga, 254u), tie_a);
        const uint32_t ub = grid_units(from(t[i]), std::min(gb, 254u), tie_b);
        if (!fl) qa = sat_add(qa, ua), qb = sat_add(qb, ub), ta |= tie_a, tb |= tie_b;
    }
    return {ga | (ta ? kTie : 0u) | flags, qa, gb | (tb ? kTie : 0u), qb};
}

bool unit_count(const Info &fu, const Grid &G, uint32_t &q) {
    const bool ok_a = (fu.meta_a & (0xffu | kTie)) == G.eg, ok_b = (fu.meta_b & (0xffu | kTie)) == G.eg;
    q = ok_a ? fu.q_a : (ok_b ? fu.q_b : 0u);
    return ok_a || ok_b;
}

// fold_chunk_terms, lane by lane: terms [0, cnt) of chunk data d, one window
// of 256 consecutive terms at a time (lane l holds terms 4 l .. 4 l + 3).
uint32_t fold_chunk_terms(Grid &G, const uint32_t *d, uint32_t cnt, bool walk, uint32_t target) {
    constexpr uint32_t kWin = 4 * kWave;
    for (uint32_t base = 0; base < kChunk && base < cnt; base += kWin) {
        uint32_t pos = 0;
        while (pos < kWin) {
            uint32_t pl[kWave][4], ties[kWave] = {}, rc[kWave], incl[kWave];
            for (uint32_t l = 0; l < kWave; ++l) {
                uint32_t run = 0;
                for (uint32_t j = 0; j < 4; ++j) {
                    const uint32_t idx = 4 * l + j;
                    const bool live = idx >= pos && base + idx < cnt;
                    bool tie;
                    const uint32_t q = grid_units(base + idx < cnt ? from(d[base + idx]) : 0.0f, G.eg, tie);
                    run += live ? q : 0u;
                    pl[l][j] = run;
                    ties[l] |= (live && tie && !g_skip_tie ? 1u : 0u) << j;
                }
                rc[l] = run < kSat ? run : kSat;
            }
            for (uint32_t l = 0, acc = 0; l < kWave; ++l) acc += rc[l], incl[l] = acc;
            bool found[kWave];
            uint32_t rv[kWave], before[kWave], tv[kWave], hj[kWave];
            for (uint32_t l = 0; l < kWave; ++l) {
                const uint32_t excl = incl[l] - rc[l];
                found[l] = false, rv[l] = 0, before[l] = excl, tv[l] = 0, hj[l] = 4;
                uint32_t prev = excl;
                for (uint32_t j = 0; j < 4; ++j) {
                    const uint32_t idx = 4 * l + j;
                    const bool live = idx >= pos && base + idx < cnt;
                    const uint32_t P = excl + pl[l][j];
                    const bool top = !g_skip_top && G.n + P >= kTop;
                    const bool vio = live && (((ties[l] >> j) & 1u) || top);
                    if (!found[l] && vio) found[l] = true, rv[l] = j, before[l] = prev, tv[l] = d[base + idx];
                    if (walk && !found[l] && live && hj[l] == 4 && grid_bits(G.eg, G.n + P) >= target) hj[l] = j;
                    prev = P;
                }
            }
            uint32_t fl = kWave, hl = kWave;
            for (uint32_t l = 0; l < kWave; ++l)
                if (found[l]) {
                    fl = l;
                    break;
                }
            if (walk) {
                for (uint32_t l = 0; l < kWave; ++l)
                    if (hj[l] < 4) {
                        hl = l;
                        break;
                    }
                if (hl < kWave && hl <= fl) return base + 4 * hl + hj[hl];
            }
            if (fl == kWave) {
                G.n += incl[kWave - 1];
                break;
            }
            const uint32_t v = 4 * fl + rv[fl];
            const float s = from(grid_bits(G.eg, G.n + before[fl])) + from(tv[fl]);
            G = grid_of(bits(s));
            if (walk && bits(s) >= target) return base + v;
            pos = v + 1;
        }
    }
    return kNoHit;
}

// fold_row: the sequential fold's value from the chunk summaries; ckpt gets
// every chunk's end value.
float fold_row(const std::vector<uint32_t> &t, const std::vector<Info> &info, std::vector<uint32_t> &ckpt) {
    const uint32_t n = (uint32_t)t.size(), nch = (uint32_t)info.size();
    uint32_t flags = 0;
    for (const Info &ci : info) flags |= ci.meta_a;
    if (flags & kNeg) {
        float s = -0.0f;
        for (uint32_t i = 0; i < n; ++i) s += from(t[i]);
        return s;
    }
    if (flags & kNan) return from(0x7fc00000u);
    if (flags & kInf) return INFINITY;
    ckpt.assign(nch, 0u);
    Grid G = {1u, 0u};
    for (uint32_t c0 = 0; c0 < nch;) {
        const uint32_t nvalid = std::min(kWave, nch - c0);
        uint32_t incl[kWave], acc = 0, fv = nvalid;
        bool vio_any = false;
        for (uint32_t l = 0; l < nvalid; ++l) {
            uint32_t q;
            const bool clean = unit_count(info[c0 + l], G, q);
            acc += clean ? q : 0u;
            incl[l] = acc;
            if (!vio_any && (!clean || G.n + incl[l] >= kTop)) vio_any = true, fv = l;
        }
        for (uint32_t l = 0; l < fv; ++l) ckpt[c0 + l] = grid_bits(G.eg, G.n + incl[l]);
        if (fv) G.n += incl[fv - 1];
        if (!vio_any) {
            c0 += nvalid;
            continue;
        }
        const uint32_t cv = c0 + fv;
        uint32_t d[kChunk] = {};
        for (uint32_t i = 0; i < kChunk && cv * kChunk + i < n; ++i) d[i] = t[cv * kChunk + i];
        fold_chunk_terms(G, d, std::min(kChunk, n - cv * kChunk), false, 0u);
        ckpt[cv] = grid_bits(G.eg, G.n);
        c0 = cv + 1;
    }
    return from(grid_bits(G.eg, G.n));
}

std::vector<Info> summaries(const std::vector<uint32_t> &t) {
    const uint32_t nch = (uint32_t)((t.size() + kChunk - 1) / kChunk);
    std::vector<double> ds(nch, 0.0);
    for (size_t i = 0; i < t.size(); ++i) ds[i / kChunk] += (double)from(t[i]);
    std::vector<Info> info(nch);
    double before = 0.0;
    for (uint32_t c = 0; c < nch; ++c) info[c] = chunk_info(t, c, before), before += ds[c];
    return info;
}

// The walk as sel_pick does it: the first group of four units whose end
// (the fold's running sum there) reaches target, then its units in order --
// a clean unit ending below target added whole, the others term by term.
uint32_t walk(const std::vector<uint32_t> &t, const std::vector<Info> &info, const std::vector<uint32_t> &ckpt,
              uint32_t target) {
    const uint32_t n = (uint32_t)t.size(), nu = (uint32_t)info.size(), ng = (nu + 3) / 4;
    uint32_t g = 0;
    while (g + 1 < ng && ckpt[std::min(4 * g + 3, nu - 1)] < target) ++g;
    Grid G = grid_of(g ? ckpt[4 * g - 1] : 0u);
    for (uint32_t u = 4 * g; u < 4 * g + 4 && u < nu; ++u) {
        uint32_t q;
        if (unit_count(info[u], G, q) && G.n + q < kTop && grid_bits(G.eg, G.n + q) < target) {
            G.n += q;
            continue;
        }
        uint32_t d[kChunk] = {};
        for (uint32_t i = 0; i < kChunk && u * kChunk + i < n; ++i) d[i] = t[u * kChunk + i];
        const uint32_t i = fold_chunk_terms(G, d, n > u * kChunk ? std::min(kChunk, n - u * kChunk) : 0u, true, target);
        if (i != kNoHit) return u * kChunk + i;
    }
    return kNoHit;
}

float seq_sum(const std::vector<uint32_t> &t) {
    volatile float s = -0.0f;  // one rounding per add, in order
    for (uint32_t w : t) s = s + from(w);
    return s;
}

uint32_t seq_walk(const std::vector<uint32_t> &t, float target) {
    volatile float cum = 0.0f;
    for (uint32_t i = 0; i < t.size(); ++i) {
        cum = cum + from(t[i]);
        if (cum >= target) return i;
    }
    return kNoHit;
}

std::vector<uint32_t> exps(const std::vector<float> &lg, float T) {
    float mx = -INFINITY;
    for (float v : lg) mx = fmaxf(mx, v);
    std::vector<uint32_t> t(lg.size());
    for (size_t i = 0; i < lg.size(); ++i) t[i] = bits(expf((lg[i] - mx) / T));
    return t;
}

std::vector<uint32_t> sorted_probs(const std::vector<uint32_t> &e) {
    const float total = seq_sum(e);
    std::vector<uint32_t> p(e.size());
    for (size_t i = 0; i < e.size(); ++i) p[i] = bits(from(e[i]) / total);
    std::stable_sort(p.begin(), p.end(), [](uint32_t a, uint32_t b) { return from(a) > from(b); });
    return p;
}

struct Tally {
    long rows = 0, mism = 0;
};

void check_row(const std::vector<uint32_t> &t, Tally &tl, std::mt19937_64 &rng, const char *what) {
    const std::vector<Info> info = summaries(t);
    std::vector<uint32_t> ckpt;
    const float got = fold_row(t, info, ckpt), want = seq_sum(t);
    ++tl.rows;
    if (bits(got) != bits(want) && !(isnan(got) && isnan(want))) {
        ++tl.mism;
        if (!g_skip_tie && !g_skip_top)
            printf("MISMATCH %s n=%zu got %a want %a\n", what, t.size(), (double)got, (double)want);
        return;
    }
    if (!isfinite(want) || !(want > 0.0f)) return;
    uint32_t flags = 0;
    for (const Info &ci : info) flags |= ci.meta_a;
    if (flags & kNeg) return;  // sel_pick walks such a row term by term (seq_walk itself)
    std::uniform_real_distribution<float> U(0.0f, 1.0f);
    for (int j = 0; j < 6; ++j) {
        const float u = j == 0 ? 0.0f : (j == 1 ? 0.99999994f : U(rng));
        const float target = u * want;
        const uint32_t a = walk(t, info, ckpt, bits(target)), b = seq_walk(t, target);
        if (a != b) {
            ++tl.mism;
            if (!g_skip_tie && !g_skip_top) printf("WALK MISMATCH %s n=%zu u=%a got %u want %u\n", what, t.size(), (double)u, a, b);
            return;
        }
    }
}

void run_all(uint64_t seed, Tally &tl) {
    std::mt19937_64 rng(seed);
    std::normal_distribution<float> N(0.0f, 1.0f);
    // the sampler's terms
    const uint32_t lens[] = {1, 2, 63, 64, 1000, 1023, 1024, 1025, 4096, 70000, 151936};
    const float scales[] = {0.1f, 1.0f, 3.0f, 30.0f};
    const float temps[] = {0.05f, 0.7f, 1.0f, 2.0f};
    for (uint32_t n : lens)
        for (float sc : scales)
            for (float T : temps) {
                if (n > 5000 && (sc == 30.0f || T == 0.05f)) continue;
                std::vector<float> lg(n);
                for (float &v : lg) v = N(rng) * sc;
                const std::vector<uint32_t> e = exps(lg, T);
                check_row(e, tl, rng, "exp");
                check_row(sorted_probs(e), tl, rng, "sorted");
            }
    // exponentials across the subnormal range
    {
        std::uniform_real_distribution<float> Ulg(-104.0f, 0.0f);
        for (uint32_t n : {2000u, 20000u}) {
            std::vector<float> lg(n);
            for (float &v : lg) v = Ulg(rng);
            const std::vector<uint32_t> e = exps(lg, 1.0f);
            check_row(e, tl, rng, "subnormal-exp");
            check_row(sorted_probs(e), tl, rng, "subnormal-sorted");
        }
    }
    // ties: 1 then many half-ulps of 1 (2^-24), of 2 (2^-23) after crossing, at both parities
    {
        std::vector<uint32_t> t = {bits(1.0f)};
        for (int i = 0; i < 3000; ++i) t.push_back(bits(i % 3 ? 0x1p-24f : 0x1.8p-23f));
        check_row(t, tl, rng, "ties");
        std::vector<uint32_t> t2 = {bits(1.0f + 0x1p-23f)};
        for (int i = 0; i < 2000; ++i) t2.push_back(bits(0x1p-24f));
        check_row(t2, tl, rng, "ties-odd");
    }
    // equal terms: sums land exactly on binade tops
    for (float v : {1.0f, 0.5f, 0x1p-130f, 0.1f, 3.0f}) {
        std::vector<uint32_t> t(5000, bits(v));
        check_row(t, tl, rng, "equal");
    }
    // jumps over several binades, and terms equal to the running sum
    {
        std::vector<uint32_t> t;
        float s = 0x1p-140f;
        for (int i = 0; i < 3000; ++i) {
            t.push_back(bits(i % 7 == 0 ? s * 37.0f : (i % 5 == 0 ? s : s * 0x1p-20f)));
            if (i % 7 == 0) s *= 8.0f;
            if (s > 1e20f) s = 0x1p-140f;
        }
        check_row(t, tl, rng, "jumps");
    }
    // random bit patterns of finite non-negative floats, over narrow and wide ranges
    for (int rep = 0; rep < 40; ++rep) {
        const uint32_t n = 1 + (uint32_t)(rng() % 9000);
        const uint32_t lo = (uint32_t)(rng() % 200), span = 1 + (uint32_t)(rng() % 40);
        std::vector<uint32_t> t(n);
        for (uint32_t &w : t) {
            const uint32_t ex = std::min(lo + (uint32_t)(rng() % span), 200u);
            w = (ex << 23) | (uint32_t)(rng() & 0x7fffffu);
            if (rng() % 50 == 0) w = 0;
        }
        check_row(t, tl, rng, "bits");
    }
    // flags: NaN, +inf, a negative term
    {
        std::vector<uint32_t> t(3000, bits(0.25f));
        t[1777] = 0x7fc00000u;
        check_row(t, tl, rng, "nan");
        t[1777] = 0x7f800000u;
        check_row(t, tl, rng, "inf");
        t[1777] = bits(-0.5f);
        check_row(t, tl, rng, "negative");
    }
}

}  // namespace

int main(int argc, char **argv) {
    const uint64_t seed = argc > 1 ? strtoull(argv[1], nullptr, 10) : 1;
    Tally tl;
    run_all(seed, tl);
    Tally ct, cp;
    g_skip_tie = true;
    run_all(seed, ct);
    g_skip_tie = false, g_skip_top = true;
    run_all(seed, cp);
    printf("rows %ld mismatches %ld control_tie %ld control_top %ld\n", tl.rows, tl.mism, ct.mism, cp.mism);
    return 0;
}
