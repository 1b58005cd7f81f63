// sxq_sample.hip -- the reference's seeded token samplers on the device, so a decode loop
// hands only a token id (not a logit row) from one step to the next.
//
//   Fish dual-AR   crates/syrinx-fish/src/common/sampling.rs: SplitMix64 (:20-37),
//                  sample_semantic (:150-163: semantic constraint + RAS),
//                  sample_codebook (:139-145: repetition penalty + nucleus),
//                  logits_to_probs (:186-240), multinomial1 (:249-263);
//   CosyVoice2/3   crates/syrinx-lm/src/cv2/sampling.rs: log_softmax_vec (:13-22),
//                  nucleus_sampling (:64-87), random_sampling (:91-95), ras_sampling
//                  (:104-124); its callers push every non-stop token into the history
//                  (crates/syrinx-lm/src/cv2/generate.rs:150-161) and the Fish driver
//                  keeps the last ras_win_size semantic ids (common/dualar.rs:188-205).
//
// One 1024-thread workgroup per stream.  Both samplers only ever draw from the top_k
// largest keys (Fish: logits; CosyVoice: probabilities), so the row is reduced on the
// device to its top_k (key, id) pairs in the reference's order -- key descending, ties by
// ascending id -- by a radix select over the ordered key bits (4 passes of 8-bit digit
// histograms, then a compaction that takes ties at the cut in id order), and the
// reference's per-candidate float steps then run on one lane in its order.
//
// A Fish draw whose top_k is 0 (unbounded, common/sampling.rs:50-52) or above the 64
// candidates one wave sorts keeps however many leading ids its top-p rule keeps: the cut is
// found by a second radix descent that carries, per digit bin, the softmax mass of its
// ids (as 2^-60 fixed-point integers, so the sums are exact and independent of the order
// of the atomics; each mass is truncated by < 2^-60, so a top-p decision can differ from
// the reference's f64 running sum only when that sum lands within ~n * 2^-60 of top_p).
// When that keeps fewer than 64 ids the wave path above runs on them (the reference's
// exact order); otherwise the whole workgroup draws over the kept ids in place: f64
// normaliser, f32 probabilities, the inverse-CDF walk in id order (sums per contiguous
// chunk of ids, then over the chunks in order).  Sums over the
// whole row (softmax normalisers, the full-distribution draw) are f64 as in the reference,
// added in a fixed tree order here rather than left to right (a difference below 1e-15
// relative, which moves a draw only when the uniform lands that close to a boundary).
// An f32 exponential is exp in f64 rounded to f32 (the correctly rounded value).
#include <math.h>

#include "../../include/sxq.h"
#include "sxq_abi.h"
#include "sxq_kernels.h"

using namespace sxq;
using namespace sxq::abi;

namespace {

constexpr int kST = 1024;        // threads per workgroup (one stream)
constexpr int kMaxTopK = 64;     // largest top_k the device samplers take
constexpr int kMaxWindow = 64;   // largest RAS window

SXQ_DEV uint64_t splitmix_next(uint64_t& state) {
    state += 0x9E3779B97F4A7C15ull;
    uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
SXQ_DEV double splitmix_f64(uint64_t& state) { return (double)(splitmix_next(state) >> 11) * (1.0 / 9007199254740992.0); }

// Ordered bits: larger float -> larger unsigned key (-inf lowest of the non-NaN values).
SXQ_DEV uint32_t order_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

SXQ_DEV float exp_f32(float x) { return (float)exp((double)x); }

// The ids a draw ranges over, in id order: [lo, hi) plus, if extra >= 0, the one id
// `extra` (outside [lo, hi)); element e -> id.
struct View {
    int lo, hi, extra;
    SXQ_DEV int count() const { return hi - lo + (extra >= 0 ? 1 : 0); }
    SXQ_DEV int id(int e) const {
        if (extra < 0) return lo + e;
        if (extra < lo) return e == 0 ? extra : lo + e - 1;
        return e < hi - lo ? lo + e : extra;
    }
};

struct Shared {
    unsigned hist[256];
    unsigned long long hmass[256];  // fixed-point softmax mass per digit bin (the top-p cut)
    float fred[kST / 64];
    double dred[kST / 64];
    unsigned wsum[kST / 64];
    float cand_key[kMaxTopK];
    int cand_id[kMaxTopK];
    float top_key[kMaxTopK];  // sorted: key descending, id ascending
    int top_id[kMaxTopK];
    double term[kMaxTopK];    // per-candidate f64 terms of a draw (by rank, then by id order)
    float prob[kMaxTopK];
    int ord[kMaxTopK];        // kept ranks in id order
    unsigned ncand;
    uint32_t kth;
    int need, result;
    double dval;
    float fval;
    unsigned long long msel;  // mass before the selected bin (the top-p cut)
};

// Inclusive prefix sum over the 64 lanes of a wave.
SXQ_DEV unsigned wave_incl_scan(unsigned x) {
    const int lane = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    return x;
}

// Exclusive prefix sum of one value per thread over the workgroup, in thread order.
SXQ_DEV unsigned block_excl_scan(unsigned v, Shared& sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const unsigned incl = wave_incl_scan(v);
    if (lane == 63) sh.wsum[wave] = incl;
    __syncthreads();
    unsigned base = 0;
    for (int w = 0; w < wave; ++w) base += sh.wsum[w];
    __syncthreads();
    return base + incl - v;
}

SXQ_DEV float block_max(float v, Shared& sh) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = sh.fred[0];
        for (int i = 1; i < kST / 64; ++i) m = fmaxf(m, sh.fred[i]);
        sh.fval = m;
    }
    __syncthreads();
    return sh.fval;
}

SXQ_DEV double block_sum(double v, Shared& sh) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) sh.dred[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = 0.0;
        for (int i = 0; i < kST / 64; ++i) s += sh.dred[i];
        sh.dval = s;
    }
    __syncthreads();
    return sh.dval;
}

// The kept set of a draw in the reference's sort order (key descending, ties by id): every
// element whose order key exceeds `key`, then the first `ties` (in id order) equal to it.
struct Cut {
    uint32_t key;
    int ties;
};

// The cut of the K largest keys of the view (K <= count) by a radix descent on counts.
template <class KeyF>
SXQ_DEV Cut count_cut(const View& v, KeyF key, int K, Shared& sh) {
    const int n = v.count(), tid = threadIdx.x;
    uint32_t prefix = 0, mask = 0;
    int rem = K;
    for (int d = 24; d >= 0; d -= 8) {
        for (int b = tid; b < 256; b += kST) sh.hist[b] = 0;
        __syncthreads();
        for (int e = tid; e < n; e += kST) {
            const uint32_t u = order_key(key(e));
            if ((u & mask) == prefix) atomicAdd(&sh.hist[(u >> d) & 0xFF], 1u);
        }
        __syncthreads();
        // the digit b where the count of keys from the top first reaches rem (b = 0 at
        // the latest): lane l of wave 0 holds digits 255 - 4l .. 252 - 4l
        if (tid < 64) {
            const int top = 255 - 4 * tid;
            const unsigned c0 = sh.hist[top], c1 = sh.hist[top - 1], c2 = sh.hist[top - 2], c3 = sh.hist[top - 3];
            const unsigned incl = wave_incl_scan(c0 + c1 + c2 + c3);
            const unsigned excl = incl - (c0 + c1 + c2 + c3);
            if ((excl < (unsigned)rem && (unsigned)rem <= incl) || (tid == 63 && incl < (unsigned)rem)) {
                unsigned above = excl;
                const unsigned c[4] = {c0, c1, c2, c3};
                int t = 0;
                for (; t < 3; ++t) {
                    if (above + c[t] >= (unsigned)rem) break;
                    above += c[t];
                }
                sh.need = rem - (int)above;  // elements of digit b still needed
                sh.kth = (uint32_t)(top - t);
            }
        }
        __syncthreads();
        prefix |= sh.kth << d;
        mask |= 0xFFu << d;
        rem = sh.need;
        __syncthreads();
    }
    return Cut{prefix, rem};
}

// The K largest keys of the view (key(e) a functor over element index), in the
// reference's sort order, into sh.top_key / sh.top_id; returns K' = min(K, count).
template <class KeyF>
SXQ_DEV int top_k_select(const View& v, KeyF key, int K, Shared& sh) {
    const int n = v.count(), tid = threadIdx.x;
    K = min(K, n);
    const Cut cut = count_cut(v, key, K, sh);
    const uint32_t prefix = cut.key;
    const int rem = cut.ties;
    // prefix = the K-th largest key; `rem` of the elements equal to it are taken, the
    // ones with the smallest ids: thread t scans the contiguous elements [t*c, t*c + c).
    const int chunk = (n + kST - 1) / kST, e0 = tid * chunk, e1 = min(n, e0 + chunk);
    if (tid == 0) sh.ncand = 0;
    unsigned ties = 0;
    for (int e = e0; e < e1; ++e) ties += order_key(key(e)) == prefix;
    unsigned rank = block_excl_scan(ties, sh);  // ties before this thread's chunk, in id order
    for (int e = e0; e < e1; ++e) {
        const float k = key(e);
        const uint32_t u = order_key(k);
        bool take = u > prefix;
        if (u == prefix) take = rank++ < (unsigned)rem;
        if (take) {
            const unsigned slot = atomicAdd(&sh.ncand, 1u);
            if (slot < (unsigned)kMaxTopK) {
                sh.cand_key[slot] = k;
                sh.cand_id[slot] = v.id(e);
            }
        }
    }
    __syncthreads();
    // rank sort of the K candidates: key descending, ties by ascending id
    if (tid < K) {
        const float k = sh.cand_key[tid];
        const int id = sh.cand_id[tid];
        const uint32_t u = order_key(k);
        int r = 0;
        for (int j = 0; j < K; ++j) {
            const uint32_t uj = order_key(sh.cand_key[j]);
            r += uj > u || (uj == u && sh.cand_id[j] < id);
        }
        sh.top_key[r] = k;
        sh.top_id[r] = id;
    }
    __syncthreads();
    return K;
}

// Fish logits_to_probs over the sorted candidates + multinomial1, run by wave 0 (every
// lane returns the token and advances its copy of rng alike).  The exponentials and
// divisions are per candidate, one lane each; the sums keep the reference's order, added
// by every lane over the shared terms: rank 0 always kept, then while cum <= top_p and
// rank < top_k (cum of exp(l - max) / total in f64, rank order); temperature softmax
// over the kept in f64 (the largest scaled key is rank 0's), probabilities rounded to f32
// and renormalised in id order; the inverse-CDF draw walks the kept ids in id order.
SXQ_DEV int fish_draw(Shared& sh, int K, double total, float mx, float temperature, float top_p, int top_k,
                      uint64_t& rng) {
    const int lane = threadIdx.x & 63;
    if (lane < K) sh.term[lane] = exp((double)(sh.top_key[lane] - mx)) / total;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    int keep = 0;
    double cum = 0.0;
    for (int r = 0; r < K; ++r) {
        if (!(r == 0 || (cum <= (double)top_p && r < top_k))) break;
        ++keep;
        cum += sh.term[r];
    }
    const float t = fmaxf(temperature, 1e-5f);
    const float kmax = sh.top_key[0] / t;
    __builtin_amdgcn_wave_barrier();
    if (lane < keep) {
        int pos = 0;
        for (int j = 0; j < keep; ++j) pos += sh.top_id[j] < sh.top_id[lane];
        sh.ord[pos] = lane;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    double e_mine = 0.0;
    if (lane < keep) {
        e_mine = exp((double)(sh.top_key[sh.ord[lane]] / t - kmax));
        sh.term[lane] = e_mine;  // id order
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    double psum = 0.0;
    for (int i = 0; i < keep; ++i) psum += sh.term[i];
    __builtin_amdgcn_wave_barrier();
    if (lane < keep) {
        float p = (float)e_mine;
        if (psum > 0.0) p = (float)((double)p / psum);
        sh.prob[lane] = p;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    double tot = 0.0;
    for (int i = 0; i < keep; ++i) tot += (double)sh.prob[i];
    if (tot <= 0.0) return 0;
    const double u = splitmix_f64(rng) * tot;
    double acc = 0.0;
    int tok = -1;  // the reference's fall-through: the row's last id (the caller maps it)
    for (int i = 0; i < keep; ++i) {
        acc += (double)sh.prob[i];
        if (u < acc) {
            tok = sh.top_id[sh.ord[i]];
            break;
        }
    }
    __builtin_amdgcn_wave_barrier();
    return tok;
}

constexpr double kFix = 1152921504606846976.0;  // 2^60: the fixed-point unit of a softmax mass

// The float whose order key is u.
SXQ_DEV float key_float(uint32_t u) { return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u); }

SXQ_DEV unsigned long long mass_q(float k, float mx, double tot) {
    return (unsigned long long)(exp((double)(k - mx)) / tot * kFix);
}

// The ids logits_to_probs keeps by its top-p rule alone -- rank 0, then every rank whose
// softmax mass before it (cum of exp(l - mx) / tot in sorted order) is <= top_p -- as a
// cut, found by a radix descent on the digit bins' fixed-point masses; `kept` = their count.
template <class KeyF>
SXQ_DEV Cut mass_cut(const View& v, KeyF key, float mx, double tot, float top_p, Shared& sh, int& kept) {
    const int n = v.count(), tid = threadIdx.x;
    if (!(top_p >= 0.0f)) {  // cum 0 > top_p: rank 0 alone
        kept = 1;
        return count_cut(v, key, 1, sh);
    }
    const unsigned long long T = top_p >= 2.0f ? (1ull << 61) : (unsigned long long)((double)top_p * kFix);
    uint32_t prefix = 0, mask = 0;
    unsigned long long above = 0;  // mass of the elements ordered before the current prefix's
    int cnt_above = 0;
    for (int d = 24; d >= 0; d -= 8) {
        for (int b = tid; b < 256; b += kST) {
            sh.hist[b] = 0;
            sh.hmass[b] = 0;
        }
        __syncthreads();
        for (int e = tid; e < n; e += kST) {
            const float k = key(e);
            const uint32_t u = order_key(k);
            if ((u & mask) == prefix) {
                const int b = (u >> d) & 0xFF;
                atomicAdd(&sh.hist[b], 1u);
                const unsigned long long q = mass_q(k, mx, tot);
                if (q) atomicAdd(&sh.hmass[b], q);
            }
        }
        __syncthreads();
        // the lowest non-empty bin whose mass before it is <= T (the non-empty bins that
        // qualify are a prefix from the top: masses only grow down the order); lane l of
        // wave 0 holds bins 255 - 4l .. 252 - 4l
        if (tid < 64) {
            const int top = 255 - 4 * tid;
            unsigned long long m[4], msum = 0;
            unsigned c[4], csum = 0;
            for (int t = 0; t < 4; ++t) {
                m[t] = sh.hmass[top - t];
                c[t] = sh.hist[top - t];
                msum += m[t];
                csum += c[t];
            }
            unsigned long long mincl = msum;
            unsigned cincl = csum;
            for (int o = 1; o < 64; o <<= 1) {
                const unsigned long long ym = __shfl_up(mincl, o, 64);
                const unsigned yc = __shfl_up(cincl, o, 64);
                if (tid >= o) {
                    mincl += ym;
                    cincl += yc;
                }
            }
            unsigned long long mb = above + (mincl - msum);
            unsigned cb = cincl - csum;
            int best = -1;
            unsigned long long best_m = 0;
            unsigned best_c = 0;
            for (int t = 0; t < 4; ++t) {
                if (c[t] && mb <= T) {
                    best = t;
                    best_m = mb;
                    best_c = cb;
                }
                mb += m[t];
                cb += c[t];
            }
            const unsigned long long has = __ballot(best >= 0);
            if (has && tid == 63 - __builtin_clzll(has)) {
                sh.kth = (uint32_t)(top - best);
                sh.need = cnt_above + (int)best_c;
                sh.msel = best_m;
            }
        }
        __syncthreads();
        prefix |= sh.kth << d;
        mask |= 0xFFu << d;
        cnt_above = sh.need;
        above = sh.msel;
        __syncthreads();
    }
    // the ties at the cut, in id order: tie j has mass above + j * q before it
    const int nties = (int)sh.hist[prefix & 0xFF];
    const unsigned long long q = mass_q(key_float(prefix), mx, tot);
    int ties = nties;
    if (q) {
        const unsigned long long j = (T - above) / q + 1;
        if (j < (unsigned long long)nties) ties = (int)j;
    }
    kept = cnt_above + ties;
    __syncthreads();
    return Cut{prefix, ties};
}

// logits_to_probs + multinomial1 over a kept set (a cut) of any size, by the whole
// workgroup: thread t takes the contiguous ids [t*c, t*c + c); the exponentials
// exp(l / t - kmax) (kmax = the view's largest key / t, rank 0's), their f64 sum, the f32
// probabilities renormalised by it and their f64 total are summed per chunk in id order,
// then over the chunks in order; the uniform's chunk is found on thread 0 and walked by
// its owner.  Only thread 0 advances rng.  Returns the id, or -1 (the reference's
// fall-through, mapped by the caller).
template <class KeyF>
SXQ_DEV int wide_draw(const View& v, KeyF key, Cut cut, float mx, float temperature, uint64_t& rng, Shared& sh,
                      double* chunk_sum) {
    const int n = v.count(), tid = threadIdx.x;
    const int chunk = (n + kST - 1) / kST, e0 = tid * chunk, e1 = min(n, e0 + chunk);
    unsigned ties = 0;
    for (int e = e0; e < e1; ++e) ties += order_key(key(e)) == cut.key;
    const unsigned tie0 = block_excl_scan(ties, sh);
    const float t = fmaxf(temperature, 1e-5f);
    const float kmax = mx / t;
    auto kept = [&](float k, unsigned& rank) {
        const uint32_t u = order_key(k);
        if (u > cut.key) return true;
        return u == cut.key && rank++ < (unsigned)cut.ties;
    };
    double ps = 0.0;
    unsigned r = tie0;
    for (int e = e0; e < e1; ++e) {
        const float k = key(e);
        if (kept(k, r)) ps += exp((double)(k / t - kmax));
    }
    chunk_sum[tid] = ps;
    __syncthreads();
    if (tid == 0) {
        double a = 0.0;
        for (int i = 0; i < kST; ++i) a += chunk_sum[i];
        sh.dval = a;
    }
    __syncthreads();
    const double psum = sh.dval;
    auto prob = [&](float k) {
        float p = (float)exp((double)(k / t - kmax));
        if (psum > 0.0) p = (float)((double)p / psum);
        return p;
    };
    double ts = 0.0;
    r = tie0;
    for (int e = e0; e < e1; ++e) {
        const float k = key(e);
        if (kept(k, r)) ts += (double)prob(k);
    }
    __syncthreads();  // psum read by every thread before chunk_sum is reused
    chunk_sum[tid] = ts;
    __syncthreads();
    if (tid == 0) {
        double total = 0.0;
        for (int i = 0; i < kST; ++i) total += chunk_sum[i];
        sh.result = -1;
        if (total <= 0.0) {
            sh.need = -1;
            sh.result = 0;  // multinomial1's empty distribution
        } else {
            const double u = splitmix_f64(rng) * total;
            double acc = 0.0;
            int c = 0;
            for (; c < kST - 1 && acc + chunk_sum[c] <= u; ++c) acc += chunk_sum[c];
            sh.need = c;
            sh.dred[0] = acc;
            sh.dval = u;
        }
    }
    __syncthreads();
    if (tid == sh.need) {
        double acc = sh.dred[0];
        r = tie0;
        for (int e = e0; e < e1; ++e) {
            const float k = key(e);
            if (!kept(k, r)) continue;
            acc += (double)prob(k);
            if (sh.dval < acc) {
                sh.result = v.id(e);
                break;
            }
        }
    }
    __syncthreads();
    const int tok = sh.result;
    __syncthreads();
    return tok;
}

// One Fish draw (logits_to_probs + multinomial1) by the whole workgroup.  kcap = the
// candidate cap (top_k, or the view's size when top_k is 0).  Up to 64 candidates: the
// top kcap are sorted and drawn on wave 0 in the reference's exact order.  A larger cap:
// the top-p cut decides how many are kept; fewer than 64 go the wave-0 way (staged one
// beyond the cut, so the exact running sum decides the last one), more are drawn in place.
// The token is returned to every thread; thread 0's rng is the advanced state.
template <class KeyF>
SXQ_DEV int block_draw(const View& v, KeyF key, float mx, double tot, float temperature, float top_p, int kcap,
                       uint64_t& rng, Shared& sh, double* chunk_sum) {
    const int tid = threadIdx.x, n = v.count();
    int K = kcap;
    if (kcap > kMaxTopK) {
        int kept = 0;
        Cut cut = mass_cut(v, key, mx, tot, top_p, sh, kept);
        if (kept >= kMaxTopK) {
            if (kept > kcap) cut = count_cut(v, key, kcap, sh);
            return wide_draw(v, key, cut, mx, temperature, rng, sh, chunk_sum);
        }
        K = min(kept + 1, n);
    }
    K = top_k_select(v, key, K, sh);
    if (tid < 64) {
        const int tok = fish_draw(sh, K, tot, mx, temperature, top_p, kcap, rng);
        if (tid == 0) sh.result = tok;
    }
    __syncthreads();
    const int tok = sh.result;
    __syncthreads();
    return tok;
}

struct FishArgs {
    const float* logits;
    int64_t stride;
    int vocab;
    sxq_fish_sampling p;
    uint64_t* rng;
    int32_t* window;
    int32_t* window_len;
    const int32_t* recent;
    int n_recent;
    int32_t* out;
    int out_stride;
    int32_t* active;  // [n] or null: a zero entry draws nothing (rng kept, out 0); a stop draw clears it
    int32_t* out2;    // a second copy of the token (null: none), out2[s * out2_stride]
    int out2_stride;
};

// mode 0: sample_semantic (constraint + RAS, window update); mode 1: sample_codebook.
template <int MODE>
__global__ __launch_bounds__(kST) void k_sample_fish(FishArgs A) {
    __shared__ Shared sh;
    __shared__ double chunk_sum[kST];
    const int s = blockIdx.x, tid = threadIdx.x;
    const float* row = A.logits + (int64_t)s * A.stride;
    const sxq_fish_sampling& P = A.p;
    if (A.active && A.active[s] == 0) {  // a finished stream: an inert 0, no draw (drive_batch)
        if (tid == 0) {
            A.out[(int64_t)s * A.out_stride] = 0;
            if (A.out2) A.out2[(int64_t)s * A.out2_stride] = 0;
        }
        return;
    }
    View v{0, A.vocab, -1};
    if (MODE == 0 && P.semantic_begin <= P.semantic_end) {
        v.lo = max(0, P.semantic_begin);
        v.hi = min(A.vocab, P.semantic_end + 1);
        v.extra = (P.stop_id >= 0 && P.stop_id < A.vocab && (P.stop_id < v.lo || P.stop_id >= v.hi)) ? P.stop_id : -1;
    }
    // the repetition penalty (codebook draws): applied per occurrence, in list order
    __shared__ float pen_val[kMaxWindow];
    __shared__ int pen_id[kMaxWindow];
    __shared__ int n_pen;
    if (tid == 0) {
        n_pen = 0;
        const bool on = MODE == 1 && A.recent && fabsf(P.repetition_penalty - 1.0f) >= 1.1920929e-07f;
        for (int i = 0; on && i < A.n_recent && i < kMaxWindow; ++i) {
            const int id = A.recent[(int64_t)s * A.n_recent + i];
            if (id < 0 || id >= A.vocab) continue;
            int j = 0;
            while (j < n_pen && pen_id[j] != id) ++j;
            float l = j < n_pen ? pen_val[j] : row[id];
            l = l > 0.0f ? l / P.repetition_penalty : l * P.repetition_penalty;
            pen_val[j] = l;
            pen_id[j] = id;
            if (j == n_pen) ++n_pen;
        }
    }
    __syncthreads();
    auto key = [&](int e) -> float {
        const int id = v.id(e);
        float l = row[id];
        if (MODE == 1)
            for (int j = 0; j < n_pen; ++j)
                if (pen_id[j] == id) l = pen_val[j];
        return l;
    };
    const int n = v.count();
    float mx = -INFINITY;
    for (int e = tid; e < n; e += kST) mx = fmaxf(mx, key(e));
    mx = block_max(mx, sh);
    double tot = 0.0;
    for (int e = tid; e < n; e += kST) tot += exp((double)(key(e) - mx));
    tot = block_sum(tot, sh);
    const int kcap = P.top_k <= 0 ? n : min(P.top_k, n);  // k_cap: 0 = unbounded
    uint64_t rng = A.rng[s];
    int tok = block_draw(v, key, mx, tot, P.temperature, P.top_p, kcap, rng, sh, chunk_sum);
    if (tok < 0) tok = A.vocab - 1;
    int high = -1;
    if (MODE == 0) {
        high = block_draw(v, key, mx, tot, P.ras_high_temp, P.ras_high_top_p, kcap, rng, sh, chunk_sum);
        if (high < 0) high = A.vocab - 1;
    }
    if (tid != 0) return;
    if (MODE == 0) {
        int* win = A.window ? A.window + (int64_t)s * P.ras_win_size : nullptr;
        // (clamped to 0..ras_win_size: a corrupt length can neither read nor write past the window)
        int len = A.window_len ? min(max(A.window_len[s], 0), P.ras_win_size) : 0;
        bool in_window = false;
        for (int i = 0; win && i < len; ++i) in_window |= win[i] == tok;
        const bool semantic = tok >= P.semantic_begin && tok <= P.semantic_end;
        if (in_window && semantic) tok = high;
        if (win && tok != P.stop_id && P.ras_win_size > 0) {  // the driver's window roll
            if (len == P.ras_win_size) {
                for (int i = 1; i < len; ++i) win[i - 1] = win[i];
                --len;
            }
            win[len++] = tok;
            A.window_len[s] = len;
        }
        if (A.active && tok == P.stop_id) A.active[s] = 0;  // is_stop: frozen from here on
    }
    A.rng[s] = rng;
    A.out[(int64_t)s * A.out_stride] = tok;
    if (A.out2) A.out2[(int64_t)s * A.out2_stride] = tok;
}

struct RasArgs {
    float* logits;
    int64_t stride;
    int vocab, ignore_eos, eos_begin, eos_end;
    float top_p, tau_r;
    int top_k, win;
    uint64_t* rng;
    int32_t* decoded;
    int32_t* decoded_len;
    int32_t* out;
    int out_stride;
};

// ras_sampling over log_softmax(logits): the row is overwritten by its log-probabilities
// (the stop ids -inf when ignore_eos), as log_softmax_vec + the mask produce them.
// Keys of the draw (the probabilities exp(log-prob), rounded to f32) kept in LDS for rows of
// up to this many ids (the CosyVoice heads: 6564 and 6761), so that the selection's six
// passes read them rather than evaluate an f64 exponential per id each time; longer rows
// recompute them.  The same values either way.
constexpr int kRasLdsKeys = 8192;

__global__ __launch_bounds__(kST) void k_sample_ras(RasArgs A) {
    __shared__ Shared sh;
    __shared__ double chunk_sum[kST];
    __shared__ float keys[kRasLdsKeys];
    __shared__ int hist_sh[kMaxWindow];
    __shared__ int hist_len;
    const int s = blockIdx.x, tid = threadIdx.x, n = A.vocab;
    float* row = A.logits + (int64_t)s * A.stride;
    // the repetition window, fetched first: its loads overlap the softmax
    if (A.decoded && tid < A.win) hist_sh[tid] = A.decoded[(int64_t)s * A.win + tid];
    if (tid == 0) hist_len = A.decoded_len ? min(max(A.decoded_len[s], 0), A.win) : 0;  // (clamped to 0..win)
    // rows of up to kRasLdsKeys ids: the row's values stay in registers for the three passes
    constexpr int kRv = kRasLdsKeys / kST;
    const bool lds_keys = n <= kRasLdsKeys;
    float rv[kRv];
    float mx = -INFINITY;
    if (lds_keys) {
#pragma unroll
        for (int j = 0; j < kRv; ++j) {
            const int i = tid + j * kST;
            rv[j] = i < n ? row[i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kRv; ++j)
            if (tid + j * kST < n) mx = fmaxf(mx, rv[j]);
    } else {
        for (int i = tid; i < n; i += kST) mx = fmaxf(mx, row[i]);
    }
    mx = block_max(mx, sh);
    double tot = 0.0;
    if (lds_keys) {
#pragma unroll
        for (int j = 0; j < kRv; ++j)
            if (tid + j * kST < n) tot += exp((double)(rv[j] - mx));
    } else {
        for (int i = tid; i < n; i += kST) tot += exp((double)(row[i] - mx));
    }
    tot = block_sum(tot, sh);
    const double lse = (double)mx + log(tot);
    if (lds_keys) {
#pragma unroll
        for (int j = 0; j < kRv; ++j) {
            const int i = tid + j * kST;
            if (i < n) {
                float lp = (float)((double)rv[j] - lse);
                if (A.ignore_eos && i >= A.eos_begin && i < A.eos_end) lp = -INFINITY;
                row[i] = lp;
                keys[i] = exp_f32(lp);
            }
        }
    } else {
        for (int i = tid; i < n; i += kST) {
            float lp = (float)((double)row[i] - lse);
            if (A.ignore_eos && i >= A.eos_begin && i < A.eos_end) lp = -INFINITY;
            row[i] = lp;
        }
    }
    __syncthreads();
    const View v{0, n, -1};
    auto key = [&](int e) -> float { return lds_keys ? keys[e] : exp_f32(row[e]); };
    const int K = top_k_select(v, key, A.top_k, sh);
    uint64_t rng = A.rng[s];
    // nucleus: the leading candidates while cum (f32) < top_p and count < top_k, drawn
    // in that (sorted) order
    if (tid == 0) {
        float cum = 0.0f;
        int c = 0;
        while (c < K && cum < A.top_p && c < A.top_k) cum += sh.top_key[c++];
        double tsum = 0.0;
        for (int i = 0; i < c; ++i) tsum += (double)sh.top_key[i];
        const double u = splitmix_f64(rng) * tsum;
        double acc = 0.0;
        int pick = c - 1;
        for (int i = 0; i < c; ++i) {
            acc += (double)sh.top_key[i];
            if (u < acc) {
                pick = i;
                break;
            }
        }
        const int top = sh.top_id[pick < 0 ? 0 : pick];
        int rep = 0;
        for (int i = 0; A.decoded && i < hist_len; ++i) rep += hist_sh[i] == top;
        sh.result = (float)rep >= (float)A.win * A.tau_r ? -1 : top;
    }
    __syncthreads();
    if (sh.result < 0) {  // random_sampling over the full distribution, ids in order
        const int chunk = (n + kST - 1) / kST, e0 = tid * chunk, e1 = min(n, e0 + chunk);
        double cs = 0.0;
        for (int i = e0; i < e1; ++i) cs += (double)key(i);
        chunk_sum[tid] = cs;
        __syncthreads();
        if (tid == 0) {
            double total = 0.0;
            for (int t = 0; t < kST; ++t) total += chunk_sum[t];
            sh.dval = splitmix_f64(rng) * total;
            double acc = 0.0;
            int t = 0;
            for (; t < kST - 1 && acc + chunk_sum[t] <= sh.dval; ++t) acc += chunk_sum[t];
            sh.need = t;        // the chunk holding the crossing
            sh.dred[0] = acc;   // the sum before that chunk
            sh.result = n - 1;  // the reference's fall-through: the last id
        }
        __syncthreads();
        if (tid == sh.need && e0 < e1) {
            double acc = sh.dred[0];
            int pick = e1 - 1;  // summed in another association than chunk_sum: stay in the chunk
            for (int i = e0; i < e1; ++i) {
                acc += (double)key(i);
                if (sh.dval < acc) {
                    pick = i;
                    break;
                }
            }
            sh.result = pick;
        }
        __syncthreads();
    }
    if (tid != 0) return;
    const int tok = sh.result;
    if (A.decoded && (tok < A.eos_begin || tok >= A.eos_end) && A.win > 0) {  // the generate loop's history
        int* hist = A.decoded + (int64_t)s * A.win;
        int len = min(max(A.decoded_len[s], 0), A.win);
        if (len == A.win) {
            for (int i = 1; i < len; ++i) hist[i - 1] = hist[i];
            --len;
        }
        hist[len++] = tok;
        A.decoded_len[s] = len;
    }
    A.rng[s] = rng;
    A.out[(int64_t)s * A.out_stride] = tok;
}

// FastAr::first_code (crates/syrinx-fish/src/s2/fast_ar.rs:105-110) per stream:
// clamp(semantic - begin, 0, residual - 1), u32 saturating at 0; an inactive stream's
// first code is the inert 0 (drive_batch's placeholder).
__global__ void k_first_codes(const int32_t* __restrict__ semantic, int sem_stride, int n, int begin, int residual,
                              const int32_t* __restrict__ active, int32_t* __restrict__ ids,
                              int32_t* __restrict__ codes, int codes_stride) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const int64_t tok = (int64_t)(uint32_t)semantic[(int64_t)s * sem_stride];
    int64_t c = tok - begin;
    c = c < 0 ? 0 : (c > residual - 1 ? residual - 1 : c);
    if (active && active[s] == 0) c = 0;
    ids[s] = (int32_t)c;
    if (codes) codes[(int64_t)s * codes_stride] = (int32_t)c;
}

// wide: the Fish draws, which take any top_k >= 0 (0 = unbounded); the CosyVoice draw
// (its reference pins top_k = 25) takes 1..64.
sxq_status check_common(int n, int vocab, int top_k, const void* logits, const void* rng, const void* out, bool wide) {
    if (n < 1 || n > 65535 || vocab < 1) return fail(SXQ_ERR_INVALID, "sample: bad shape (%d streams, %d ids)", n, vocab);
    if (wide ? top_k < 0 : (top_k < 1 || top_k > kMaxTopK))
        return fail(SXQ_ERR_INVALID, wide ? "sample: top_k %d is negative" : "sample: top_k %d outside 1..%d on the device",
                    top_k, kMaxTopK);
    if (!logits || !rng || !out) return fail(SXQ_ERR_INVALID, "sample: null pointer");
    return SXQ_OK;
}

}  // namespace

namespace sxq {
namespace abi {

bool fish_sampling_fits(const sxq_fish_sampling& p) { return p.top_k >= 0; }

hipError_t launch_sample_codebook(const float* logits, int64_t stride, int n, int vocab, const sxq_fish_sampling& p,
                                  uint64_t* rng, const int32_t* active, int32_t* out, int out_stride, int32_t* out2,
                                  int out2_stride, hipStream_t s) {
    FishArgs A{logits, stride, vocab, p, rng, nullptr, nullptr, nullptr, 0, out, out_stride,
               const_cast<int32_t*>(active), out2, out2_stride};
    hipLaunchKernelGGL(k_sample_fish<1>, dim3(n), dim3(kST), 0, s, A);
    return hipGetLastError();
}

hipError_t launch_first_codes(const int32_t* semantic, int sem_stride, int n, int begin, int residual,
                              const int32_t* active, int32_t* ids, int32_t* codes, int codes_stride, hipStream_t s) {
    hipLaunchKernelGGL(k_first_codes, dim3((n + 63) / 64), dim3(64), 0, s, semantic, sem_stride, n, begin, residual,
                       active, ids, codes, codes_stride);
    return hipGetLastError();
}

}  // namespace abi
}  // namespace sxq

extern "C" {

sxq_status sxq_sample_semantic(int device, const float* logits, int64_t logits_stride, int n, int vocab,
                               const sxq_fish_sampling* p, uint64_t* rng, int32_t* window, int32_t* window_len,
                               int32_t* active, int32_t* out, int out_stride, void* stream) {
    if (!p) return fail(SXQ_ERR_INVALID, "sample_semantic: null parameters");
    sxq_status st = check_common(n, vocab, p->top_k, logits, rng, out, true);
    if (st != SXQ_OK) return st;
    if (p->ras_win_size < 0 || p->ras_win_size > kMaxWindow)
        return fail(SXQ_ERR_INVALID, "sample_semantic: ras_win_size %d outside 0..%d", p->ras_win_size, kMaxWindow);
    if (!window != !window_len) return fail(SXQ_ERR_INVALID, "sample_semantic: window and window_len go together");
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    FishArgs A{logits, logits_stride, vocab, *p, rng, window, window_len, nullptr, 0, out, out_stride, active, nullptr, 0};
    hipLaunchKernelGGL(k_sample_fish<0>, dim3(n), dim3(kST), 0, (hipStream_t)stream, A);
    HIP_TRY(hipGetLastError(), "sample_semantic");
    return SXQ_OK;
}

sxq_status sxq_sample_codebook(int device, const float* logits, int64_t logits_stride, int n, int vocab,
                               const sxq_fish_sampling* p, uint64_t* rng, const int32_t* recent, int n_recent,
                               const int32_t* active, int32_t* out, int out_stride, void* stream) {
    if (!p) return fail(SXQ_ERR_INVALID, "sample_codebook: null parameters");
    sxq_status st = check_common(n, vocab, p->top_k, logits, rng, out, true);
    if (st != SXQ_OK) return st;
    if (n_recent < 0 || n_recent > kMaxWindow || (n_recent > 0 && !recent))
        return fail(SXQ_ERR_INVALID, "sample_codebook: %d recent ids (at most %d)", n_recent, kMaxWindow);
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    FishArgs A{logits, logits_stride, vocab, *p, rng, nullptr, nullptr, recent, n_recent, out, out_stride,
               const_cast<int32_t*>(active), nullptr, 0};
    hipLaunchKernelGGL(k_sample_fish<1>, dim3(n), dim3(kST), 0, (hipStream_t)stream, A);
    HIP_TRY(hipGetLastError(), "sample_codebook");
    return SXQ_OK;
}

sxq_status sxq_sample_ras(int device, float* logits, int64_t logits_stride, int n, int vocab, int ignore_eos,
                          int eos_begin, int eos_end, float top_p, int top_k, int win, float tau_r, uint64_t* rng,
                          int32_t* decoded, int32_t* decoded_len, int32_t* out, int out_stride, void* stream) {
    sxq_status st = check_common(n, vocab, top_k, logits, rng, out, false);
    if (st != SXQ_OK) return st;
    if (win < 0 || win > kMaxWindow) return fail(SXQ_ERR_INVALID, "sample_ras: window %d outside 0..%d", win, kMaxWindow);
    if (!decoded != !decoded_len) return fail(SXQ_ERR_INVALID, "sample_ras: decoded and decoded_len go together");
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    RasArgs A{logits, logits_stride, vocab, ignore_eos, eos_begin, eos_end, top_p, tau_r, top_k, win, rng, decoded,
              decoded_len, out, out_stride};
    hipLaunchKernelGGL(k_sample_ras, dim3(n), dim3(kST), 0, (hipStream_t)stream, A);
    HIP_TRY(hipGetLastError(), "sample_ras");
    return SXQ_OK;
}

}  // extern "C"
