// sxq_attn_dev.h -- fused GQA decode attention of one split as a device function:
// QK-norm + RoPE + KV append + split partials + last-arriver merge + quantization of
// the context (the kernel is k_attn_decode in sxq_decoder.hip).
//
// Reference: crates/syrinx-fish/src/s2/nn.rs:325-352 (QK-norm, RoPE, KV append,
// attention), crates/syrinx-lm/src/cv2/attention.rs:67-88; f32 throughout as on the
// reference CPU path.
#pragma once
#include "sxq_decoder.h"
#include "sxq_quant_dev.h"
#include "sxq_sync_dev.h"

namespace sxq {

// Copy rows [0, n) of a K and a V tile (row stride hd floats in global memory, hd + 4 in
// LDS) with every thread's loads of a batch in flight together -- the LDS stores wait
// for the whole batch rather than for each load in turn.  256 threads.
SXQ_DEV void load_kv_tile(float* kt, float* vt, const float* kb, const float* vb, int n, int hd) {
    constexpr int kBatch = 8;  // float4 of K and of V per thread per batch
    const int hd4 = hd / 4, n4 = n * hd4, hdp = hd + 4;
    for (int base = 0; base < n4; base += 256 * kBatch) {
        float4 kv[kBatch], vv[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int i = min(base + j * 256 + (int)threadIdx.x, n4 - 1);  // clamped: in bounds
            const int p = i / hd4, d4 = i - p * hd4;
            kv[j] = *(const float4*)(kb + (int64_t)p * hd + 4 * d4);
            vv[j] = *(const float4*)(vb + (int64_t)p * hd + 4 * d4);
        }
        // An empty asm reading every loaded register: the loads cannot be sunk to their
        // stores (each would then wait for its own load); they are all issued first and
        // the stores below wait once for the batch.  It emits no instruction.
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            asm volatile("" ::"v"(kv[j].x), "v"(kv[j].y), "v"(kv[j].z), "v"(kv[j].w), "v"(vv[j].x), "v"(vv[j].y),
                         "v"(vv[j].z), "v"(vv[j].w));
        // clamped like the loads (unconditional, so no branch pulls a load down to its
        // store): out-of-range threads rewrite the last row element with its own value
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int i = min(base + j * 256 + (int)threadIdx.x, n4 - 1);
            const int p = i / hd4, d4 = i - p * hd4;
            *(float4*)(kt + p * hdp + 4 * d4) = kv[j];
            *(float4*)(vt + p * hdp + 4 * d4) = vv[j];
        }
    }
}

struct RopeIn {
    float a, b, wa, wb, c, sn;
};
// Loads for one head's norm + RoPE: lane i < HD/2 owns the pair (2i, 2i+1) interleaved or
// (i, i + HD/2) rotate-half.  No branch around the loads (lanes past HD/2 repeat a pair,
// masked in rope_finish; without norm weights the source is loaded in their place), so
// the compiler's wait for them counts only the loads issued after them.
template <int HD>
SXQ_DEV RopeIn rope_load(const float* src, const float* nw, int interleaved, const float* cos_row,
                         const float* sin_row, int lane) {
    const int i = lane & (HD / 2 - 1);
    const int ia = interleaved ? 2 * i : i, ib = interleaved ? 2 * i + 1 : i + HD / 2;
    const float* w = nw ? nw : src;
    RopeIn r;
    r.a = src[ia];
    r.b = src[ib];
    r.wa = w[ia];
    r.wb = w[ib];
    r.c = cos_row[i];
    r.sn = sin_row[i];
    return r;
}
// y = RoPE(norm(x)) for the pair loaded by rope_load, in registers: no LDS access and no
// branch (without norm the scale is exactly 1), so it runs while the loads issued after
// rope_load are still in flight.  Wave-uniform control flow (the norm's sum of squares
// is a wave reduction).
template <int HD>
SXQ_DEV float2 rope_pair(const RopeIn& r, bool norm, float eps, float inv_hd, int lane) {
    const bool own = lane < HD / 2;
    float a = own ? r.a : 0.0f, b = own ? r.b : 0.0f;
    const float ss = wave_sum_rows(a * a + b * b);
    const float den = norm ? sqrtf((ss * inv_hd + 0.0f) * 1.0f + eps) : 1.0f;
    a = (a / den) * (norm ? r.wa : 1.0f);
    b = (b / den) * (norm ? r.wb : 1.0f);
    return make_float2(a * r.c - b * r.sn, b * r.c + a * r.sn);
}
// Stores the pair from rope_pair (lanes < HD/2) to dst[] and, if non-null, gdst[].
template <int HD>
SXQ_DEV void rope_store(float2 y, int interleaved, float* dst, float* gdst, int lane) {
    if (lane < HD / 2) {
        const int ia = interleaved ? 2 * lane : lane, ib = interleaved ? 2 * lane + 1 : lane + HD / 2;
        dst[ia] = y.x;
        dst[ib] = y.y;
        if (gdst) {
            gdst[ia] = y.x;
            gdst[ib] = y.y;
        }
    }
}

// The group's context slice (thread t < T holds elements 4t .. 4t + 3, zeros past T): the
// optional f32 record, then the activation blocks of the O projection -- the quantizers'
// lane layout, wave w quantizing chunk w of 256 elements.
// PUB: the slice is read by other workgroups of the same launch (the O projection of
// k_attn_wo_decode), so it is quantized into LDS at smem + A.pub_off bytes, copied out
// by wave 0 with agent-coherent 16-byte stores and, once those have completed, counted
// in every copy of A.ready.
template <int VDT, int HD, bool PUB = false>
SXQ_DEV void attn_emit_context(const AttnArgs& A, int s, int g, int gd, int T, float4 v, float* smem) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int dim = A.nh * HD;
    if (tid < T && A.ctx_out) *(float4*)(A.ctx_out + (int64_t)s * dim + (int64_t)g * gd + 4 * tid) = v;
    const int nbr = VDT == kQ8K ? dim / 256 : dim / 32;  // activation blocks per row
    uint8_t* arow = A.act + (int64_t)s * nbr * act_block_bytes(VDT);
    const int blk_first = VDT == kQ8K ? (g * gd) / 256 : (g * gd) / 32;  // the slice's first block
    uint8_t* qdst = arow + (size_t)blk_first * act_block_bytes(VDT);
    if constexpr (PUB) {
        uint8_t* ql = (uint8_t*)smem + A.pub_off;
        if (tid < ((T + 63) & ~63)) {
            if constexpr (VDT == kQ8K)
                wave_quantize_q8k<false>(v, lane, ql + (size_t)wave * sizeof(ActQ8K));
            else
                wave_quantize_q8_0<false>(v, lane, wave * 8 + (lane >> 3) < gd / 32, ql + (size_t)wave * 8 * sizeof(ActQ8_0));
        }
        lds_barrier();
        if (wave == 0) {
            const int nu4 = VDT == kQ8K ? (gd / 256) * (int)(sizeof(ActQ8K) / 16) : (gd / 32) * (int)(sizeof(ActQ8_0) / 16);
            const __amdgpu_buffer_rsrc_t r = coherent_rsrc(qdst, (uint32_t)nu4 * 16);
            for (int i = lane; i < nu4; i += 64) store16_coherent(r, (uint32_t)i * 16, ((const float4*)ql)[i]);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the slice has reached the coherent level
            if (lane < A.ready_copies)  // every copy of the counter
                __hip_atomic_fetch_add(A.ready + lane * A.cstride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    if (tid < ((T + 63) & ~63)) {
        if (VDT == kQ8K)
            wave_quantize_q8k<false>(v, lane, qdst + (size_t)wave * sizeof(ActQ8K), A.rec ? A.rec + blk_first + wave : nullptr,
                                     s);
        else
            wave_quantize_q8_0<false>(v, lane, wave * 8 + (lane >> 3) < gd / 32, qdst + (size_t)wave * 8 * sizeof(ActQ8_0));
    }
}

typedef float attn_v4f __attribute__((ext_vector_type(4)));  // (HIP's float4 array would go to scratch)

// The key tile of split sp (P = NT/8 positions) into registers: 8 lanes per position,
// 16-byte pieces 32 floats apart, so every load instruction reads whole 128-byte rows;
// rows past the stream's last position (L - 1) clamped to it (loaded, never used).
template <int HD, int NT>
SXQ_DEV void attn_load_k(float4 (&kr)[HD / 32], const AttnArgs& A, int64_t head_off, int sp, int L) {
    constexpr int P = NT / 8;
    const int tid = threadIdx.x, p0 = sp * P, slot = min(P, L - p0) - 1;
    const int kp = tid >> 3, kcol = 4 * (tid & 7);
    const float* krow = A.kc + head_off + (int64_t)(p0 + min(kp, slot)) * HD + kcol;
#pragma unroll
    for (int j = 0; j < HD / 32; ++j) kr[j] = ld_global((const float4*)(krow + 32 * j));
}
// The value tile of split sp, coalesced: round r holds floats [r*4NT, r*4NT + 4NT) of the
// tile, 4 per thread.  In the split holding position L - 1 (the last of the nsp) that row
// is the new value, read from the qkv row.  (Register loads, not direct-to-LDS ones: with
// a direct-to-LDS load in flight the compiler waits for every load before the first use
// of any.)
template <int HD, int NT>
SXQ_DEV void attn_load_v(attn_v4f (&vr4)[HD / 32], const AttnArgs& A, int64_t head_off, const float* vrow_new, int sp,
                         int L, int nsp) {
    constexpr int P = NT / 8, VR = P * HD / (4 * NT);
    static_assert(VR == HD / 32, "NT = 8 P");
    const int tid = threadIdx.x, p0 = sp * P, slot = min(P, L - p0) - 1;
    const bool has_new = sp == nsp - 1;
    const float* vb = A.vc + head_off + (int64_t)p0 * HD;
#pragma unroll
    for (int r = 0; r < VR; ++r) {
        const int e = r * 4 * NT + 4 * tid;
        const int vr = min(e / HD, slot), col = e - (e / HD) * HD;
        const float* src = has_new && vr == slot ? vrow_new + col : vb + (int64_t)vr * HD + col;
        vr4[r] = ld_global((const attn_v4f*)src);
    }
}

// The loads of a split issued before the stream's length is known (SPEC, batch 1): the
// length (a scalar load, so waiting for it does not wait for the vector loads), the
// norm + RoPE inputs with the step's RoPE row (A.rope_row: cos then sin at the stream's
// position, copied by the step's embedding kernel), then the key and value tiles of all
// P positions (rows clamped to the cache; rows past the length are never read: the
// softmax masks their scores and the weighted values stop at the length).  Wave w
// loads item min(w, G): a query head, or the new key from wave G on (used only by the
// split holding the position); with G == NW wave 0 also loads the new key as rin2.
template <int HD>
struct SplitLoads {
    RopeIn rin, rin2;
    int item;
    float4 kr[HD / 32];
    attn_v4f vr4[HD / 32];
};
template <int HD, int NT, int GC>
SXQ_DEV int attn_spec_loads(SplitLoads<HD>& R, const AttnArgs& A, int s, int g, int sp) {
    constexpr int P = NT / 8, NW = NT / 64, VR = HD / 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = A.len[s];
    issue_point();  // the length's load first
    const int nh = A.nh, G = GC > 0 ? GC : nh / A.nkv;
    const float* row = A.qkv + (int64_t)s * A.qkv_n;
    const float *cr = A.rope_row, *sr = A.rope_row + HD / 2;
    R.item = min(wave, G);
    const bool isq = R.item < G;
    R.rin = rope_load<HD>(row + (int64_t)(isq ? g * G + R.item : nh + g) * HD, isq ? A.qn : A.kn, A.interleaved, cr, sr,
                          lane);
    if (G == NW && wave == 0) R.rin2 = rope_load<HD>(row + (int64_t)(nh + g) * HD, A.kn, A.interleaved, cr, sr, lane);
    const int64_t head_off = (int64_t)s * A.kv_stream_stride + (int64_t)g * A.max_seq * HD;
    const int p0 = sp * P, last = A.max_seq - 1;
    {
        const int kp = tid >> 3, kcol = 4 * (tid & 7);
        const float* krow = A.kc + head_off + (int64_t)min(p0 + kp, last) * HD + kcol;
#pragma unroll
        for (int j = 0; j < HD / 32; ++j) R.kr[j] = ld_global((const float4*)(krow + 32 * j));
    }
#pragma unroll
    for (int r = 0; r < VR; ++r) {
        const int e = r * 4 * NT + 4 * tid, vr = e / HD, col = e - vr * HD;
        R.vr4[r] = ld_global((const attn_v4f*)(A.vc + head_off + (int64_t)min(p0 + vr, last) * HD + col));
    }
    issue_point();
    return pos;
}

// The partials of one split of the fused decode attention, NT threads: split sp of KV
// head group g of stream s, P = NT/8 cached positions [sp*P, sp*P + P) (the stream holds
// pos + 1 positions in nsp splits), leaving the split's partials {m, l, 0, 0, acc[hd]}
// per head
//   m = max_j s_j, l = sum_j exp(s_j - m), acc = sum_j exp(s_j - m) v_j,  s_j = (q . k_j) * scale
// in part_s -- or, when one split holds every position, the group's context itself.
// QK-norm + RoPE of the group's G queries (from the qkv row) and, in the split holding
// position pos, of the new token's key, appended to the cache with its value.  Returns
// true when the caller is to publish the partials (nsp > 1).
//
// Latency layout (a launch holds ~B * n_kv * L / P workgroups, about one per CU at batch
// 1, so every phase is a chain of dependent steps rather than a throughput problem):
//   * the loads of each wave's norm + RoPE item (wave h: query head h; wave G: the new
//     key) go first, then the key tile and the value tile, so the norm + RoPE runs while
//     the tiles are in flight;
//   * scores: each lane dots its key elements with the same elements of every query
//     (LDS broadcast), reduced over its 8 lanes with DPP; the value tile goes to LDS
//     after them (it is first read by the weighted values);
//   * softmax: a wave per head, positions lane + 64 i, DPP reductions;
//   * weighted values: nq = NT / (G*HD/4) position sets, a thread per (set, head, 4
//     columns), the sets summed in order through LDS.
// The barriers are LDS-only (lds_barrier): no global access inside the split is read
// back by another thread of the workgroup (the partials are published after it).
template <int VDT, int HD, int NT, int GC, bool PUB = false>
SXQ_DEV bool attn_split(const AttnArgs& A, int s, int g, int sp, int pos, int nsp, float* smem, float* part_s,
                        __amdgpu_buffer_rsrc_t prs, SplitLoads<HD>* pre = nullptr) {
    constexpr int P = NT / 8, KJ = HD / 32, PR = HD + 4, NW = NT / 64, VR = HD / 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = pos + 1, p0 = sp * P;
    const int nh = A.nh, nkv = A.nkv, max_splits = A.max_splits;
    const int np = min(P, L - p0);
    const int G = GC > 0 ? GC : nh / nkv, gd = G * HD, T = gd / 4, nq = NT / T;
    const bool has_new = sp == nsp - 1;  // position pos is then row np - 1 of the tile
    const int slot = np - 1;
    float* vt = smem;            // [P][HD]   value tile
    float* knew = vt + P * HD;   // [HD]      the new key after QK-norm + RoPE
    float* sc = knew + HD;       // [G][P]    scores, then exp(s - m)
    float* qs = sc + G * P;      // [G][HD]   queries after QK-norm + RoPE (read by the scores)
    float* red = qs;             // [nq-1][gd] weighted sums of position sets 1.. (written after
                                 //            the scores; set 0's stay in its threads' registers)
    const float* row = A.qkv + (int64_t)s * A.qkv_n;
    const float* cos_row = A.cos_t + (int64_t)pos * (HD / 2);
    const float* sin_row = A.sin_t + (int64_t)pos * (HD / 2);
    const int64_t head_off = (int64_t)s * A.kv_stream_stride + (int64_t)g * A.max_seq * HD;
    const float* vrow_new = row + (int64_t)(nh + nkv + g) * HD;
    const int kp = tid >> 3, kcol = 4 * (tid & 7);

    // 1. this wave's norm + RoPE item (every wave loads one; idle waves repeat the last),
    //    then the key and value tiles -- or, from the loads issued before the length
    //    (pre), the same with the new value's row put in place
    const int nitem = G + (has_new ? 1 : 0);
    const int item = pre ? pre->item : min(wave, nitem - 1);
    const bool isq = item < G;
    const float* inw = isq ? A.qn : A.kn;
    RopeIn rin;
    float4 kr[KJ];
    attn_v4f vr4[VR];
    if (pre) {
        rin = pre->rin;
#pragma unroll
        for (int j = 0; j < KJ; ++j) kr[j] = pre->kr[j];
#pragma unroll
        for (int r = 0; r < VR; ++r) {
            vr4[r] = pre->vr4[r];
            const int e = r * 4 * NT + 4 * tid, vr = e / HD;
            if (has_new && vr == slot) vr4[r] = ld_global((const attn_v4f*)(vrow_new + (e - vr * HD)));
        }
    } else {
        rin = rope_load<HD>(row + (int64_t)(isq ? g * G + item : nh + g) * HD, inw, A.interleaved, cos_row, sin_row,
                            lane);
        attn_load_k<HD, NT>(kr, A, head_off, sp, L);
        attn_load_v<HD, NT>(vr4, A, head_off, vrow_new, sp, L, nsp);
        issue_point();
    }
    // 2. norm + RoPE in registers while the tiles are in flight
    {
        float2 y = rope_pair<HD>(rin, inw != nullptr, A.eps, A.inv_hd, lane);
        float2 y2 = make_float2(0.0f, 0.0f);
        if (wave + NW < nitem) {  // G == NW: the new key is a second item of wave 0
            const RopeIn r2 = pre ? pre->rin2
                                  : rope_load<HD>(row + (int64_t)(nh + g) * HD, A.kn, A.interleaved, cos_row, sin_row, lane);
            y2 = rope_pair<HD>(r2, A.kn != nullptr, A.eps, A.inv_hd, lane);
        }
        float* kapp = A.kc + head_off + (int64_t)pos * HD;  // the new key's cache row
        if (wave < nitem)
            rope_store<HD>(y, A.interleaved, isq ? qs + item * HD : knew,
                           isq ? (A.q_out && sp == 0 ? A.q_out + ((int64_t)s * nh + g * G + item) * HD : nullptr) : kapp,
                           lane);
        if (wave + NW < nitem) rope_store<HD>(y2, A.interleaved, knew, kapp, lane);
        lds_barrier();
    }
    if (has_new && kp == slot)
#pragma unroll
        for (int j = 0; j < KJ; ++j) kr[j] = *(const float4*)(knew + kcol + 32 * j);
    // 3. scores: partial dots over this lane's key elements, summed over the 8 lanes of the
    //    position; lane c of the 8 writes head c's score
    float sv[8];
#pragma unroll
    for (int h = 0; h < 8; ++h) {
        float acc = 0.0f;
        if (h < G) {
#pragma unroll
            for (int j = 0; j < KJ; ++j) {
                const float4 q = *(const float4*)(qs + h * HD + kcol + 32 * j);
                acc += q.x * kr[j].x;
                acc += q.y * kr[j].y;
                acc += q.z * kr[j].z;
                acc += q.w * kr[j].w;
            }
            acc += dpp_f32<0xB1>(acc);
            acc += dpp_f32<0x4E>(acc);
            acc += dpp_f32<0x141>(acc);
        }
        sv[h] = acc;
    }
    const int c8 = tid & 7;
    float mine = sv[0];
#pragma unroll
    for (int h = 1; h < 8; ++h)
        if (c8 == h) mine = sv[h];
    if (c8 < G) sc[c8 * P + kp] = mine * A.scale + 0.0f;
    // the value tile into LDS (it is first read by the weighted values)
#pragma unroll
    for (int r = 0; r < VR; ++r) *(attn_v4f*)(vt + r * 4 * NT + 4 * tid) = vr4[r];
    lds_barrier();
    if (has_new && wave == NW - 1)  // append the new value to the cache
#pragma unroll
        for (int t = 0; t < HD / 64; ++t)
            A.vc[head_off + (int64_t)pos * HD + lane + 64 * t] = vt[slot * HD + lane + 64 * t];
    // 4. softmax of head `wave` over the tile's positions (lane + 64 i)
    if (wave < G) {
        constexpr int PL = P / 64;
        float x[PL], mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            x[i] = lane + 64 * i < np ? sc[wave * P + lane + 64 * i] : -INFINITY;
            mx = fmaxf(mx, x[i]);
        }
        const float m = wave_max_rows(mx);
        float ls = 0.0f;
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            const float e = lane + 64 * i < np ? expf(x[i] - m) : 0.0f;
            sc[wave * P + lane + 64 * i] = e;
            ls += e;
        }
        const float l = wave_sum_rows(ls);
        if (lane == 0) {
            if (nsp == 1) {
                knew[wave] = l;  // (the new key is in kr by now)
            } else {
                float* pm = part_s + ((int64_t)(g * G + wave) * max_splits + sp) * PR;
                store_agent(pm, m);
                store_agent(pm + 1, l);
            }
        }
    }
    lds_barrier();
    // 5. weighted values: thread (set qi, head h, columns d..d+3) over the set's positions
    const int pps = (P + nq - 1) / nq;
    const int qi = tid / T, rr = tid - qi * T, h = rr / (HD / 4), d = 4 * (rr - h * (HD / 4));
    float4 own = make_float4(0.0f, 0.0f, 0.0f, 0.0f);  // set 0: thread tid < T holds elements 4 tid..
    if (qi < nq) {
        const int pa = qi * pps, pb = min(pa + pps, np);
        const float* e = sc + h * P;
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
        for (int p = pa; p < pb; ++p) {
            const float w = e[p];
            const float4 v = *(const float4*)(vt + p * HD + d);
            a.x += w * v.x;
            a.y += w * v.y;
            a.z += w * v.z;
            a.w += w * v.w;
        }
        if (qi == 0) own = a;
        else *(float4*)(red + (qi - 1) * gd + h * HD + d) = a;
    }
    lds_barrier();
    if (nsp == 1) {
        // One split holds every position: its weights exp(m - m) are 1, so the merge
        // would give acc / l bit for bit -- without the hand-off.
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (tid < T) {
            float4 a = own;
            for (int q = 1; q < nq; ++q) {
                const float4 b = *(const float4*)(red + (q - 1) * gd + 4 * tid);
                a.x += b.x;
                a.y += b.y;
                a.z += b.z;
                a.w += b.w;
            }
            const float ls = knew[(4 * tid) / HD];
            v = make_float4(a.x / ls, a.y / ls, a.z / ls, a.w / ls);
        }
        attn_emit_context<VDT, HD, PUB>(A, s, g, gd, T, v, smem);
        return false;
    }
    if (tid < T) {
        float4 a = own;
        for (int q = 1; q < nq; ++q) {
            const float4 b = *(const float4*)(red + (q - 1) * gd + 4 * tid);
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        store16_coherent(prs, (uint32_t)(((g * G + h) * max_splits + sp) * PR + 4 + d) * 4, a);
    }
    return true;
}

// Fused decode attention for split sp of KV head group g of stream s (attn_split),
// then, in the last split of the group to finish (a per-(stream, group) arrival
// counter, reset after use), the merge of the group's heads and the quantization of that
// G*hd slice of the context for the O projection.
//   merge: the same (set, head, 4 columns) threads as the weighted values read their
//   splits' partials with 16-byte coherent loads issued together, the split weights
//   formed meanwhile.
// Requires HD in {64, 128}, G <= 8 and G*HD a whole number of activation blocks; GC is
// G as a compile-time constant (the Qwen3-4B and Qwen2-0.5B groups), or 0 to read it
// from A at run time.
template <int VDT, int HD, int NT, int GC, bool PUB = false, bool SPEC = false>
SXQ_DEV void attn_decode_body(const AttnArgs& A, int s, int g, int sp, float* smem, bool* last) {
    constexpr int P = NT / 8, PR = HD + 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    SplitLoads<HD> R;
    const int pos = SPEC ? attn_spec_loads<HD, NT, GC>(R, A, s, g, sp) : A.len[s], nsp = (pos + P) / P;
    if (sp >= nsp) return;
    const int nh = A.nh, nkv = A.nkv, max_splits = A.max_splits;
    const int G = GC > 0 ? GC : nh / nkv, gd = G * HD, T = gd / 4, nq = NT / T;
    float* part_s = A.part + (int64_t)s * nh * max_splits * PR;
    const __amdgpu_buffer_rsrc_t prs = coherent_rsrc(part_s, (uint32_t)nh * (uint32_t)max_splits * PR * 4);
    if (!attn_split<VDT, HD, NT, GC, PUB>(A, s, g, sp, pos, nsp, smem, part_s, prs, SPEC ? &R : nullptr)) return;
    // the last split of the group to arrive merges the group's heads
    if (!publish_and_count(&A.counter[(s * nkv + g) * A.cstride], (unsigned)nsp, last)) return;

    // merge: ctx = sum_z exp(m_z - M) acc_z / sum_z exp(m_z - M) l_z, M = max_z m_z.
    // The tile LDS is free now: wts [G][nsp] | lsum [G] | red2 [nq][gd].
    const int qi = tid / T, rr = tid - qi * T, h = rr / (HD / 4), d = 4 * (rr - h * (HD / 4));
    const bool mt = qi < nq;
    float* wts = smem;
    float* lsum = wts + G * nsp;
    float* red2 = smem + ((G * nsp + G + 3) & ~3);
    // m and l of every split first (wave h < G, lane i: splits i, i + 64, ...)...
    constexpr int kRounds = kMaxSplitsFused / 64;
    float mv[kRounds], lv[kRounds];
    if (wave < G) {
        const float* ph = part_s + (int64_t)(g * G + wave) * max_splits * PR;
#pragma unroll
        for (int c = 0; c < kRounds; ++c) {
            const int i = min(lane + 64 * c, nsp - 1);  // clamped: in bounds, masked below
            mv[c] = load_agent(ph + (int64_t)i * PR);
            lv[c] = load_agent(ph + (int64_t)i * PR + 1);
        }
    }
    // ... then this thread's partials, splits z = qi + nq*b, kMergeBatch at a time
    constexpr int kMergeBatch = 8;
    const int zper = (nsp + nq - 1) / nq;  // splits per set, rounded up (uniform)
    const uint32_t rec0 = (uint32_t)((g * G + h) * max_splits) * PR * 4 + (uint32_t)(4 + d) * 4;
    float4 pv[kMergeBatch];
#pragma unroll
    for (int b = 0; b < kMergeBatch; ++b) {
        const int z = min(qi + nq * b, nsp - 1);
        pv[b] = load16_coherent(prs, rec0 + (uint32_t)z * PR * 4);
    }
    if (wave < G) {
        float M = -INFINITY;
#pragma unroll
        for (int c = 0; c < kRounds; ++c)
            if (lane + 64 * c < nsp) M = fmaxf(M, mv[c]);
        M = wave_max_rows(M);
        float Ls = 0.0f;
#pragma unroll
        for (int c = 0; c < kRounds; ++c) {
            const int i = lane + 64 * c;
            if (i < nsp) {
                const float w = expf(mv[c] - M);
                wts[wave * nsp + i] = w;
                Ls += lv[c] * w;
            }
        }
        Ls = wave_sum_rows(Ls);
        if (lane == 0) lsum[wave] = Ls;
    }
    __syncthreads();
    float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int b0 = 0; b0 < zper; b0 += kMergeBatch) {
        if (b0 > 0)
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b) {
                const int z = min(qi + nq * (b0 + b), nsp - 1);
                pv[b] = load16_coherent(prs, rec0 + (uint32_t)z * PR * 4);
            }
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b) {
            const int z = qi + nq * (b0 + b);
            if (mt && z < nsp) {
                const float w = wts[h * nsp + z];
                a.x += pv[b].x * w;
                a.y += pv[b].y * w;
                a.z += pv[b].z * w;
                a.w += pv[b].w * w;
            }
        }
    }
    if (mt) *(float4*)(red2 + qi * gd + h * HD + d) = a;
    __syncthreads();
    // 8. context: thread t < T holds elements 4t .. 4t + 3 of the group's slice
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (tid < T) {
        float4 c = *(const float4*)(red2 + 4 * tid);
        for (int q = 1; q < nq; ++q) {
            const float4 b = *(const float4*)(red2 + q * gd + 4 * tid);
            c.x += b.x;
            c.y += b.y;
            c.z += b.z;
            c.w += b.w;
        }
        const float ls = lsum[(4 * tid) / HD];
        v = make_float4(c.x / ls, c.y / ls, c.z / ls, c.w / ls);
    }
    attn_emit_context<VDT, HD, PUB>(A, s, g, gd, T, v, smem);
    if (tid == 0) __hip_atomic_store(&A.counter[(s * nkv + g) * A.cstride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace sxq
