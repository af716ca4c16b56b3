// Segment-aware GAE / returns as a reverse affine scan, and masked whitening,
// for gfx950.
//
// The recursion of _reverse_scan_reference (meshy/backend/titan/critic/gae.py:162-180)
//     A_t = x_t + decay_t * cont_t * A_{t+1},   A = 0 outside valid
// is a composition of affine maps f_t(A) = a_t * A + b_t with a_t = decay_t *
// cont_t and b_t = x_t (zero outside valid).  cont_t (gae.py:77-93) is 0 at
// the end of each row, at a document change and at a mask hole, so the whole
// [rows, S] grid is one flattened sequence and no segment bookkeeping is
// needed beyond a_t = 0.  Maps compose as (p1, q1) o (p2, q2) = (p1 p2, q1 + p1 q2):
//   k_gae_doc_count / k_gae_count  masked token count per document
//                (index_add, gae.py:264-269), only when lengths are not given:
//                one workgroup per document over its segment offsets, a
//                fixed-order sum (bitwise reproducible), when the caller
//                passes the offsets of non-decreasing ids; otherwise fp32
//                atomics (exact for 0/1 masks);
//   k_gae_scan   one pass, workgroup b on chunk nc - 1 - b (right to left):
//                folds its chunk of kChunk tokens into one map per scan
//                (advantages and returns) and publishes it in the chunk's
//                slot, folds its carry-in from the slots of the chunks to its
//                right up to the first one that cuts both scans (both slopes
//                exactly 0: nothing past it reaches the chunk), waiting for
//                slots not yet published, then scans its threads from the
//                right seeded with the carry and writes A_t and G_t from the
//                inputs it holds in registers; it also writes lambda per
//                document (gae.py:70-74);
//   k_gae_fix    returns at once unless the call held a non-finite term (or
//                a wait was given up): then it redoes the outputs from the
//                slots, composing with hardness, as the reference's loop
//                carries a NaN across document ends.
// With the segment offsets of non-decreasing ids, a chunk holding at most
// kMaxStarts document starts reads the ids only at its two ends and takes the
// starts from the offsets (8 bytes per token less); other chunks read every
// token's id.
// Every fold of the scan has a fixed order, so the results do not depend on
// timing (the atomic count aside).
// Everything is fp32, like the reference's sequential fallback.
#include <algorithm>
#include <atomic>

#include "common.h"

namespace meshy {
namespace {

constexpr int kThreads = 256;
constexpr int kItems = 8;
constexpr int64_t kChunk = static_cast<int64_t>(kThreads) * kItems;
static_assert(kItems % 8 == 0 || kItems == 4, "bf16 values are loaded 8 (or 4) at a time");
constexpr int64_t kXcds = 8;        // workgroups go round-robin over the XCDs
constexpr int kCountThreads = 256;
constexpr int kCountItems = 16;

struct Aff {
    float p, q;  // A_before = p * A_after + q
};

// A map with slope -0 is "hard": it ignores its input, as the recursion does at
// a row end, where each row of the reference's [rows, S] grid starts afresh.
// Every other slope is >= +0 (gamma >= 0), so a product of slopes is never -0
// by itself.  A soft cut (a document end or a mask hole, slope +0) still passes
// a NaN or infinite input on, since 0 * NaN and 0 * inf are NaN in the
// reference's sequential loop; a hard one does not.
__device__ __forceinline__ bool is_hard(float p) { return __float_as_uint(p) == 0x80000000u; }

// left covers earlier positions than right.  kHard: hard if either is, and a
// hard left map ignores the right one.  Without kHard, plain composition: the
// same values whenever every input is finite (a row end's slope is a zero
// either way), and cheaper; the kernels take it unless the call holds a
// non-finite term.
template <bool kHard>
__device__ __forceinline__ Aff compose(Aff left, Aff right) {
    if constexpr (kHard) {
        const bool hl = is_hard(left.p);
        const bool h = hl || is_hard(right.p);
        return Aff{h ? -0.f : left.p * right.p, hl ? left.q : fmaf(left.p, right.q, left.q)};
    } else {
        return Aff{left.p * right.p, fmaf(left.p, right.q, left.q)};
    }
}

// The map applied to a value: a hard map ignores it.
template <bool kHard>
__device__ __forceinline__ float apply_map(Aff f, float x) {
    if constexpr (kHard) return is_hard(f.p) ? f.q : fmaf(f.p, x, f.q);
    return fmaf(f.p, x, f.q);
}

// Set (atomic max) by k_gae_scan to the call's epoch when some chunk holds a
// non-finite term (a NaN or infinite advantage or return term at a valid
// position) or a wait for a neighbour's map was given up.  k_gae_fix then
// redoes the call, composing with hardness and folding each carry up to the
// row's end instead of stopping at the first cut, which a non-finite value
// crosses in the reference.  Epochs grow per call, so no clearing is needed
// and calls on other streams can only send a call down the slower, exact path.
__device__ unsigned long long g_gae_nonfinite_epoch = 0;

struct Pair {
    Aff adv, ret;
};
template <bool kHard>
__device__ __forceinline__ Pair compose(const Pair& l, const Pair& r) {
    return Pair{compose<kHard>(l.adv, r.adv), compose<kHard>(l.ret, r.ret)};
}
__device__ __forceinline__ Pair identity_pair() { return Pair{Aff{1.f, 0.f}, Aff{1.f, 0.f}}; }

// A chunk's published map: four 64-bit words (adv.p, adv.q, ret.p, ret.q),
// each the float's bits in the low half and in the high half a tag drawn from
// the call, the chunk and the word.  Each word is stored and loaded as one
// single-copy atomic, so a reader takes a word as published exactly when its
// tag is the call's: words left from an earlier call (or any other data the
// workspace held) carry other tags, so nothing is cleared between calls.
// A slot is accepted only when all four tags match.
struct Slot {
    unsigned long long w[4];
};

struct Workspace {
    float* cnt;     // [n_docs + 1]
    Slot* slot;     // [n_chunks]
};

int64_t n_chunks_of(int64_t n) { return (n + kChunk - 1) / kChunk; }

size_t ws_bytes(int64_t n, int64_t n_docs) {
    const int64_t nc = n_chunks_of(n);
    return align_up(sizeof(float) * (n_docs + 1), 256) + align_up(sizeof(Slot) * nc, 256);
}

Workspace ws_of(void* base, int64_t n, int64_t n_docs) {
    char* p = static_cast<char*>(base);
    Workspace w;
    w.cnt = reinterpret_cast<float*>(p);
    p += align_up(sizeof(float) * (n_docs + 1), 256);
    w.slot = reinterpret_cast<Slot*>(p);
    return w;
}

// The tag of word w of chunk c's slot in call `call` (a 64-bit mix).
__device__ __forceinline__ uint32_t slot_tag(unsigned long long call, int64_t c, int w) {
    unsigned long long x = call * 0x9E3779B97F4A7C15ull +
                           (static_cast<unsigned long long>(c) * 4 + static_cast<unsigned>(w)) * 0xBF58476D1CE4E5B9ull;
    x ^= x >> 31;
    x *= 0x94D049BB133111EBull;
    x ^= x >> 29;
    return static_cast<uint32_t>(x >> 32);
}

__device__ __forceinline__ unsigned long long tagged(float v, unsigned long long call, int64_t c, int w) {
    return (static_cast<unsigned long long>(slot_tag(call, c, w)) << 32) | __float_as_uint(v);
}

// Loads at device (agent) scope: they see stores other XCDs made during this
// launch, whatever the loading XCD's L2 holds.
__device__ __forceinline__ unsigned long long load_word(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float word_value(unsigned long long x) {
    return __uint_as_float(static_cast<uint32_t>(x));
}

// Chunk k's map if all four words of its slot carry the call's tags.
__device__ __forceinline__ bool read_slot(const Slot* slots, int64_t k, unsigned long long call, Pair& out) {
    const unsigned long long a = load_word(&slots[k].w[0]);
    const unsigned long long b = load_word(&slots[k].w[1]);
    const unsigned long long c = load_word(&slots[k].w[2]);
    const unsigned long long d = load_word(&slots[k].w[3]);
    const bool ok = static_cast<uint32_t>(a >> 32) == slot_tag(call, k, 0) &&
                    static_cast<uint32_t>(b >> 32) == slot_tag(call, k, 1) &&
                    static_cast<uint32_t>(c >> 32) == slot_tag(call, k, 2) &&
                    static_cast<uint32_t>(d >> 32) == slot_tag(call, k, 3);
    out = Pair{Aff{word_value(a), word_value(b)}, Aff{word_value(c), word_value(d)}};
    return ok;
}

// Chunk k's map after the launch that published it has ended (the tags are
// not checked).
__device__ __forceinline__ Pair slot_pair(const Slot* slots, int64_t k) {
    const Slot s = slots[k];
    return Pair{Aff{word_value(s.w[0]), word_value(s.w[1])}, Aff{word_value(s.w[2]), word_value(s.w[3])}};
}

__device__ __forceinline__ float lambda_of(float L, float alpha, float epsilon) {
    // _lambda_per_doc: clamp(1 - 1/(alpha * max(L, 1)), 0, 1 - epsilon)
    const float lam = 1.f - 1.f / (alpha * fmaxf(L, 1.f));
    return fminf(fmaxf(lam, 0.f), 1.f - epsilon);
}

__device__ __forceinline__ float doc_length(const meshy_gae_args& g, const float* cnt, int64_t d) {
    return g.lengths ? g.lengths[d] : cnt[d];
}

__device__ __forceinline__ float value_at(const meshy_gae_args& g, int64_t t) {
    if (!g.values) return 0.f;
    if (g.values_bf16) return bf16_to_f32(static_cast<const uint16_t*>(g.values)[t]);
    return static_cast<const float*>(g.values)[t];
}

// The inputs of a thread's kItems positions plus the next one (its neighbour
// in time), loaded with 16-byte vector loads when the run is whole and aligned.
struct ThreadInputs {
    float mk[kItems + 1];
    int64_t d[kItems + 1];
    float v[kItems + 1];
    float r[kItems];
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef long long i64x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// The documents of a chunk's window [c0, e), e = min(c0 + kChunk + 1, n) (the
// chunk and the neighbour of its last position), from the ids at its two ends
// and the offsets of the document starts between them, so that the per-token
// ids are not read.  Used with offsets, both end ids in [0, n_docs] and at most
// kMaxStarts starts inside; otherwise the chunk reads every token's id.
constexpr int kMaxStarts = 4;

struct ChunkDocs {
    int64_t d0;                  // the id at c0
    int64_t start[kMaxStarts];   // first position of documents d0 + 1, ... (INT64_MAX past the last)
    bool use;
};

// A load at a workgroup-uniform address of data the kernel does not write,
// through the scalar unit: it waits on its own counter, not behind the
// vector loads issued before it.
__device__ __forceinline__ int64_t load_scalar(const int64_t* p) {
    return *(const __attribute__((address_space(4))) int64_t*)(p);
}

__device__ __forceinline__ ChunkDocs chunk_docs(const meshy_gae_args& g, int64_t c0, int64_t n) {
    ChunkDocs cd;
    cd.use = false;
    cd.d0 = 0;
#pragma unroll
    for (int r = 0; r < kMaxStarts; ++r) cd.start[r] = INT64_MAX;
    if (!g.seg_offsets || c0 >= n) return cd;
    const int64_t e = min(c0 + kChunk + 1, n);
    const int64_t d0 = load_scalar(g.doc_ids + c0);
    const int64_t d1 = load_scalar(g.doc_ids + e - 1);
    if (d0 < 0 || d1 > g.n_docs || d1 < d0 || d1 - d0 > kMaxStarts) return cd;
    cd.use = true;
    cd.d0 = d0;
#pragma unroll
    for (int r = 0; r < kMaxStarts; ++r)
        if (r < d1 - d0) cd.start[r] = load_scalar(g.seg_offsets + d0 + 1 + r);
    return cd;
}

// The id at position t of the chunk's window (non-decreasing ids: the starts at
// or before t, empty documents included, each add one).
__device__ __forceinline__ int64_t id_in_chunk(const ChunkDocs& cd, int64_t t) {
    int64_t d = cd.d0;
#pragma unroll
    for (int r = 0; r < kMaxStarts; ++r) d += (t >= cd.start[r]) ? 1 : 0;
    return d;
}

// Mask, rewards and values of the thread's kItems positions and the next one
// (its neighbour in time), with 16-byte vector loads when the run is whole
// and aligned.
__device__ __forceinline__ void load_tokens(const meshy_gae_args& g, int64_t t0, int64_t n, bool vec,
                                            ThreadInputs& in) {
    const bool whole = vec && t0 + kItems <= n;
    if (whole) {
#pragma unroll
        for (int q = 0; q < kItems / 4; ++q) {
            const f32x4 m4 = *reinterpret_cast<const f32x4*>(g.mask + t0 + 4 * q);
            const f32x4 r4 = *reinterpret_cast<const f32x4*>(g.rewards + t0 + 4 * q);
            in.mk[4 * q + 0] = m4.x; in.mk[4 * q + 1] = m4.y; in.mk[4 * q + 2] = m4.z; in.mk[4 * q + 3] = m4.w;
            in.r[4 * q + 0] = r4.x; in.r[4 * q + 1] = r4.y; in.r[4 * q + 2] = r4.z; in.r[4 * q + 3] = r4.w;
        }
        if (g.values) {
            if (g.values_bf16) {
                const uint16_t* vb = static_cast<const uint16_t*>(g.values) + t0;
                if constexpr (kItems % 8 == 0) {
#pragma unroll
                    for (int q = 0; q < kItems / 8; ++q) {
                        const u32x4 w = *reinterpret_cast<const u32x4*>(vb + 8 * q);
                        in.v[8 * q + 0] = bf16_lo(w.x); in.v[8 * q + 1] = bf16_hi(w.x);
                        in.v[8 * q + 2] = bf16_lo(w.y); in.v[8 * q + 3] = bf16_hi(w.y);
                        in.v[8 * q + 4] = bf16_lo(w.z); in.v[8 * q + 5] = bf16_hi(w.z);
                        in.v[8 * q + 6] = bf16_lo(w.w); in.v[8 * q + 7] = bf16_hi(w.w);
                    }
                } else {
                    const u32x2 w = *reinterpret_cast<const u32x2*>(vb);
                    in.v[0] = bf16_lo(w.x); in.v[1] = bf16_hi(w.x);
                    in.v[2] = bf16_lo(w.y); in.v[3] = bf16_hi(w.y);
                }
            } else {
                const float* vf = static_cast<const float*>(g.values) + t0;
#pragma unroll
                for (int q = 0; q < kItems / 4; ++q) {
                    const f32x4 v4 = *reinterpret_cast<const f32x4*>(vf + 4 * q);
                    in.v[4 * q + 0] = v4.x; in.v[4 * q + 1] = v4.y; in.v[4 * q + 2] = v4.z; in.v[4 * q + 3] = v4.w;
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < kItems; ++k) in.v[k] = 0.f;
        }
    } else {
#pragma unroll
        for (int k = 0; k < kItems; ++k) {
            const int64_t t = t0 + k;
            const bool ok = t < n;
            in.mk[k] = ok ? g.mask[t] : 0.f;
            in.r[k] = ok ? g.rewards[t] : 0.f;
            in.v[k] = ok ? value_at(g, t) : 0.f;
        }
    }
    const int64_t tn = t0 + kItems;
    const bool okn = tn < n;
    in.mk[kItems] = okn ? g.mask[tn] : 0.f;
    in.v[kItems] = okn ? value_at(g, tn) : 0.f;
}

// Every position's id from doc_ids (-1 past n).
__device__ __forceinline__ void load_ids(const meshy_gae_args& g, int64_t t0, int64_t n, bool vec,
                                         ThreadInputs& in) {
    if (vec && t0 + kItems <= n) {
#pragma unroll
        for (int q = 0; q < kItems / 2; ++q) {
            const i64x2 d2 = *reinterpret_cast<const i64x2*>(g.doc_ids + t0 + 2 * q);
            in.d[2 * q] = d2.x;
            in.d[2 * q + 1] = d2.y;
        }
    } else {
#pragma unroll
        for (int k = 0; k < kItems; ++k) in.d[k] = (t0 + k < n) ? g.doc_ids[t0 + k] : -1;
    }
    const int64_t tn = t0 + kItems;
    in.d[kItems] = tn < n ? g.doc_ids[tn] : -1;
}

// The thread's inputs: the token loads first, then the chunk's documents
// (scalar loads, which do not wait behind them), then the ids, from the
// chunk's starts when it has them, else from doc_ids.  The branch on cd.use is
// uniform over the workgroup.
__device__ __forceinline__ void load_inputs(const meshy_gae_args& g, int64_t c0, int64_t t0, int64_t n, bool vec,
                                            ThreadInputs& in) {
    load_tokens(g, t0, n, vec, in);
    const ChunkDocs cd = chunk_docs(g, c0, n);
    if (cd.use) {
#pragma unroll
        for (int k = 0; k <= kItems; ++k) in.d[k] = (t0 + k < n) ? id_in_chunk(cd, t0 + k) : -1;
    } else {
        load_ids(g, t0, n, vec, in);
    }
}

// The affine maps of a thread's positions t0 .. t0 + kItems - 1 (identity past n).
// Row ends come from a column counter started with one division; lambda is
// recomputed only when the document changes.
__device__ __forceinline__ void thread_maps(const meshy_gae_args& g, const float* cnt, int64_t c0, int64_t t0,
                                            int64_t n, bool vec, Pair (&items)[kItems], uint32_t& valid_bits,
                                            bool& has_row_end) {
    ThreadInputs in;
    load_inputs(g, c0, t0, n, vec, in);
    int64_t s = t0 % g.S;
    int64_t cur_d = -2;
    float cur_lam = 0.f;
    valid_bits = 0;
    has_row_end = false;
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        if (t0 + k >= n) {
            items[k] = identity_pair();
            continue;
        }
        const bool row_end = (s == g.S - 1);
        has_row_end |= row_end;
        s = row_end ? 0 : s + 1;
        const float mk = in.mk[k];
        const bool valid = mk > 0.f;
        const int64_t d = in.d[k];
        const bool cont = valid && !row_end && in.d[k + 1] == d && in.mk[k + 1] > 0.f;
        const float vn = row_end ? 0.f : in.v[k + 1];
        if (d != cur_d) {
            cur_d = d;
            // The padding slot (and any id outside [0, n_docs)) gets lambda 0.
            cur_lam = (d >= 0 && d < g.n_docs) ? lambda_of(doc_length(g, cnt, d), g.alpha, g.epsilon) : 0.f;
        }
        const float contf = cont ? 1.f : 0.f;
        const float validf = valid ? 1.f : 0.f;
        const float r = in.r[k];
        const float delta = (r + g.gamma * vn * contf - in.v[k]) * validf;
        items[k].adv = Aff{row_end ? -0.f : (g.gamma * cur_lam) * contf, valid ? delta : 0.f};
        items[k].ret = Aff{row_end ? -0.f : g.gamma * contf, valid ? r : 0.f};
        valid_bits |= valid ? (1u << k) : 0u;
    }
}

// DPP moves (checked on the device): row_shl:N, lane l reads lane l + N of its
// 16-lane row; wave_shl:1, lane l reads lane l + 1 of the wave.  A lane whose
// source lies past the row's (wave's) end keeps its own value.
constexpr int kDppRowShl1 = 0x101, kDppRowShl2 = 0x102, kDppRowShl4 = 0x104, kDppRowShl8 = 0x108;
constexpr int kDppWaveShl1 = 0x130;

template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

template <int kCtrl>
__device__ __forceinline__ Pair dpp_pair(const Pair& v) {
    return Pair{Aff{dpp_mov<kCtrl>(v.adv.p), dpp_mov<kCtrl>(v.adv.q)},
                Aff{dpp_mov<kCtrl>(v.ret.p), dpp_mov<kCtrl>(v.ret.q)}};
}

__device__ __forceinline__ Pair lane_pair(const Pair& v, int l) {
    return Pair{Aff{lane_f32(v.adv.p, l), lane_f32(v.adv.q, l)}, Aff{lane_f32(v.ret.p, l), lane_f32(v.ret.q, l)}};
}

// Composition of the 64 lanes' maps in lane order (lane 0 leftmost), as a
// fixed tree: pairs, quads, eights and sixteens within each row through DPP
// shifts (lanes 0, 16, 32, 48 then hold their row's fold), then
// (row 0 o row 1) o (row 2 o row 3) from those lanes.  The result is in
// every lane.  All 64 lanes must be active.
template <bool kHard>
__device__ __forceinline__ Pair wave_fold(Pair x) {
    x = compose<kHard>(x, dpp_pair<kDppRowShl1>(x));
    x = compose<kHard>(x, dpp_pair<kDppRowShl2>(x));
    x = compose<kHard>(x, dpp_pair<kDppRowShl4>(x));
    x = compose<kHard>(x, dpp_pair<kDppRowShl8>(x));
    return compose<kHard>(compose<kHard>(lane_pair(x, 0), lane_pair(x, 16)),
                          compose<kHard>(lane_pair(x, 32), lane_pair(x, 48)));
}

// Suffix composition across the block (lane order, lane 0 leftmost): for each
// thread the map of all items of the threads after it (exclusive), and the
// block total.  Within each 16-lane row a scan through DPP row shifts (lane l
// then holds its row's suffix from l); the rows' folds, read from lanes 0, 16,
// 32 and 48, complete each lane's suffix to the wave's end; the waves meet in
// LDS.  All 64 lanes of every wave must be active.
template <bool kHard>
__device__ __forceinline__ Pair block_suffix_exclusive(Pair mine, Pair* s_wave, Pair& total) {
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
    const int rl = lane % 16;
    constexpr int kW = kThreads / kWave;
    Pair incl = mine;
    {
        const Pair o = dpp_pair<kDppRowShl1>(incl);
        incl = rl + 1 < 16 ? compose<kHard>(incl, o) : incl;
    }
    {
        const Pair o = dpp_pair<kDppRowShl2>(incl);
        incl = rl + 2 < 16 ? compose<kHard>(incl, o) : incl;
    }
    {
        const Pair o = dpp_pair<kDppRowShl4>(incl);
        incl = rl + 4 < 16 ? compose<kHard>(incl, o) : incl;
    }
    {
        const Pair o = dpp_pair<kDppRowShl8>(incl);
        incl = rl + 8 < 16 ? compose<kHard>(incl, o) : incl;
    }
    const Pair r0 = lane_pair(incl, 0);
    const Pair r3 = lane_pair(incl, 48);
    const Pair a1 = compose<kHard>(lane_pair(incl, 32), r3);  // rows 2, 3
    const Pair a0 = compose<kHard>(lane_pair(incl, 16), a1);  // rows 1, 2, 3
    const int row = lane / 16;
    const Pair after_row = row == 0 ? a0 : (row == 1 ? a1 : (row == 2 ? r3 : identity_pair()));
    incl = compose<kHard>(incl, after_row);  // lane l .. lane 63
    if (lane == 0) s_wave[wid] = compose<kHard>(r0, a0);  // whole-wave map
    __syncthreads();
    Pair after_wave = identity_pair();
    for (int w = kW - 1; w > wid; --w) after_wave = compose<kHard>(s_wave[w], after_wave);
    total = identity_pair();
    for (int w = kW - 1; w >= 0; --w) total = compose<kHard>(s_wave[w], total);
    __syncthreads();
    // exclusive within the wave = inclusive of the next lane
    const Pair next = dpp_pair<kDppWaveShl1>(incl);
    return lane + 1 < kWave ? compose<kHard>(next, after_wave) : after_wave;
}

__global__ __launch_bounds__(kThreads) void k_gae_zero(float* p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

__global__ __launch_bounds__(kCountThreads) void k_gae_count(meshy_gae_args g, float* cnt, int64_t n) {
    const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * kCountThreads + threadIdx.x) * kCountItems;
    if (t0 >= n) return;
    const int64_t t1 = min(t0 + kCountItems, n);
    int64_t cur = g.doc_ids[t0];
    float acc = 0.f;
    for (int64_t t = t0; t < t1; ++t) {
        const int64_t d = g.doc_ids[t];
        if (d != cur) {
            if (cur >= 0 && cur <= g.n_docs && acc != 0.f) atomicAdd(cnt + cur, acc);
            cur = d;
            acc = 0.f;
        }
        acc += g.mask[t];
    }
    if (cur >= 0 && cur <= g.n_docs && acc != 0.f) atomicAdd(cnt + cur, acc);
}

// Masked token count of document blockIdx.x over its offsets range: every
// thread sums a fixed set of positions (four loads in flight), then a
// fixed-order block sum; the result does not depend on timing.
__global__ __launch_bounds__(kCountThreads) void k_gae_doc_count(const float* __restrict__ mask,
                                                                 const int64_t* __restrict__ off,
                                                                 float* __restrict__ cnt) {
    __shared__ float s_red[kCountThreads / kWave];
    const int64_t d = blockIdx.x;
    const int64_t lo = off[d];
    const int64_t hi = off[d + 1];
    float acc = 0.f;
    int64_t t = lo + threadIdx.x;
    for (; t + 3 * kCountThreads < hi; t += 4 * kCountThreads) {
        const float a0 = mask[t], a1 = mask[t + kCountThreads], a2 = mask[t + 2 * kCountThreads],
                    a3 = mask[t + 3 * kCountThreads];
        acc += (a0 + a1) + (a2 + a3);
    }
    for (; t < hi; t += kCountThreads) acc += mask[t];
    acc = block_sum<kCountThreads>(acc, s_red);
    if (threadIdx.x == 0) cnt[d] = acc;
}

// The thread's maps (contiguous positions) folded right to left.
template <bool kHard>
__device__ __forceinline__ Pair fold_items(const Pair (&items)[kItems]) {
    Pair agg = identity_pair();
#pragma unroll
    for (int k = kItems - 1; k >= 0; --k) agg = compose<kHard>(items[k], agg);
    return agg;
}

// The chunk's map, composed in every wave (each wave folds the waves' maps from
// LDS, so every thread holds the result).
template <bool kHard>
__device__ __forceinline__ Pair chunk_map(const Pair (&items)[kItems], Pair* s_wave) {
    const Pair wf = wave_fold<kHard>(fold_items<kHard>(items));
    if (threadIdx.x % kWave == 0) s_wave[threadIdx.x / kWave] = wf;
    __syncthreads();
    Pair total = identity_pair();
    for (int w = kThreads / kWave - 1; w >= 0; --w) total = compose<kHard>(s_wave[w], total);
    return total;
}

// The chunk's map for the slots.  A plain fold is NaN or infinite exactly
// when one of its terms is (0 * NaN, 0 * inf and NaN + x are all NaN), so the
// plain map tells whether the chunk holds a non-finite term; only then is the
// map composed again with hardness.  A plain map takes its hardness (a row end
// in the chunk) from the positions.  Every thread returns the same map.
__device__ __forceinline__ Pair published_map(const Pair (&items)[kItems], bool has_row_end, Pair* s_wave,
                                              Pair* s_wave_hard, int* s_row_end, bool& nonfinite) {
    const bool wave_row_end = __ballot(has_row_end) != 0;
    if (threadIdx.x % kWave == 0) s_row_end[threadIdx.x / kWave] = wave_row_end;
    Pair total = chunk_map<false>(items, s_wave);  // its barrier publishes s_row_end
    nonfinite = !isfinite(total.adv.q) || !isfinite(total.ret.q);
    if (nonfinite) return chunk_map<true>(items, s_wave_hard);
    bool hard = false;
    for (int w = 0; w < kThreads / kWave; ++w) hard |= s_row_end[w] != 0;
    if (hard) {
        total.adv.p = -0.f;
        total.ret.p = -0.f;
    }
    return total;
}

__device__ __forceinline__ void write_lambda(const meshy_gae_args& g, const float* cnt, int64_t first, int64_t step) {
    // Lambda per document (gae.py:271-275), reported to the caller.
    for (int64_t d = first; d < g.n_docs; d += step) g.lam_doc[d] = lambda_of(doc_length(g, cnt, d), g.alpha, g.epsilon);
}

__global__ __launch_bounds__(kThreads) void k_gae_lambda(meshy_gae_args g, const float* cnt) {
    write_lambda(g, cnt, static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x,
                 static_cast<int64_t>(gridDim.x) * kThreads);
}

// The chunk's outputs from its carry-in (s_carry, written by wave 0 before
// the call): scans the threads from the right seeded with the carry and
// writes A_t and G_t.
template <bool kHard>
__device__ __forceinline__ void scan_and_write(const meshy_gae_args& g, int64_t n, bool vec, int64_t c,
                                               Pair* s_suffix, const float* s_carry, const Pair (&items)[kItems],
                                               uint32_t valid_bits) {
    const int64_t t0 = c * kChunk + static_cast<int64_t>(threadIdx.x) * kItems;
    const Pair mine = fold_items<kHard>(items);
    Pair total;
    const Pair excl = block_suffix_exclusive<kHard>(mine, s_suffix, total);  // its barriers publish s_carry
    float A = apply_map<kHard>(excl.adv, s_carry[0]);
    float G = apply_map<kHard>(excl.ret, s_carry[1]);
    float outA[kItems], outG[kItems];
#pragma unroll
    for (int k = kItems - 1; k >= 0; --k) {
        A = apply_map<kHard>(items[k].adv, A);
        G = apply_map<kHard>(items[k].ret, G);
        // Zero outside valid (gae.py:180), whatever the recursion carries there.
        const bool valid = (valid_bits >> k) & 1u;
        outA[k] = valid ? A : 0.f;
        outG[k] = valid ? G : 0.f;
    }
    if (vec && t0 + kItems <= n) {
#pragma unroll
        for (int q = 0; q < kItems / 4; ++q) {
            if (g.adv)
                *reinterpret_cast<f32x4*>(g.adv + t0 + 4 * q) =
                    f32x4{outA[4 * q], outA[4 * q + 1], outA[4 * q + 2], outA[4 * q + 3]};
            if (g.returns)
                *reinterpret_cast<f32x4*>(g.returns + t0 + 4 * q) =
                    f32x4{outG[4 * q], outG[4 * q + 1], outG[4 * q + 2], outG[4 * q + 3]};
        }
    } else {
#pragma unroll
        for (int k = 0; k < kItems; ++k) {
            if (t0 + k < n) {
                if (g.adv) g.adv[t0 + k] = outA[k];
                if (g.returns) g.returns[t0 + k] = outG[k];
            }
        }
    }
}

// Polls of one batch of slots before a wait is given up (each poll is a
// round trip to memory and a short sleep: about 2-4 ms in all).  A chunk only
// waits for chunks to its right, whose workgroups come earlier in the grid, so
// every wait is expected to end; one given up leaves the call to k_gae_fix.
constexpr int kMaxPolls = 2000;
// Slots in a chunk's first batch: most chunks find a cut among their first
// few neighbours, and polling 64 slots at once from every workgroup loads the
// memory system (1024-document workload: 35.9 us per call with 64, 28.9 with
// 4, 29.4 with 2); later batches take 64.
constexpr int kFirstBatch = 4;

// One pass: workgroup b takes chunk c = nc - 1 - b (the grid runs right to
// left), folds it to its map and publishes it in the chunk's slot, then wave 0
// folds the carry-in from the slots of the chunks to its right, in order, up
// to and including the first whose map cuts both scans (both slopes exactly
// 0: a document end, a row end or a mask hole lies in it).  With p = 0,
// (p, q) o (p', q') = (0, q) for any finite q', so nothing past that chunk
// reaches the carry; the maps come kFirstBatch, then 64 at a time (one
// wave_fold per batch, composed in order), a ballot finds the first cut
// and one DPP fold covers the lanes up to it, a fixed order whatever the
// timing.  A slot not yet published is polled again.  Then the chunk rescans
// itself from registers (each input is read once) and writes A and G; the grid
// also writes lambda per document.
// Everything composes plainly: the same values as composing with hardness
// when every term is finite.  A chunk holding a non-finite term, or a wait
// given up, records the call's epoch in g_gae_nonfinite_epoch and k_gae_fix
// redoes the call's outputs.
__global__ __launch_bounds__(kThreads) void k_gae_scan(meshy_gae_args g, Workspace ws, int64_t n, int64_t nc,
                                                       bool vec, unsigned long long epoch, int max_polls) {
    // The chunk map and the suffix scan use separate arrays: a wave may enter
    // the scan while another still reads the map's array.
    __shared__ Pair s_wave[kThreads / kWave];
    __shared__ Pair s_wave_hard[kThreads / kWave];
    __shared__ Pair s_suffix[kThreads / kWave];
    __shared__ int s_row_end[kThreads / kWave];
    __shared__ float s_carry[2];
    const int64_t c = nc - 1 - static_cast<int64_t>(blockIdx.x);
    const int lane = threadIdx.x % kWave;
    Pair items[kItems];
    uint32_t valid_bits;
    bool has_row_end;
    thread_maps(g, ws.cnt, c * kChunk, c * kChunk + static_cast<int64_t>(threadIdx.x) * kItems, n, vec, items,
                valid_bits, has_row_end);
    bool nonfinite;
    const Pair total = published_map(items, has_row_end, s_wave, s_wave_hard, s_row_end, nonfinite);
    if (threadIdx.x < 4) {
        const float v = threadIdx.x == 0 ? total.adv.p
                        : threadIdx.x == 1 ? total.adv.q
                        : threadIdx.x == 2 ? total.ret.p
                                           : total.ret.q;
        if (nonfinite && threadIdx.x == 0) atomicMax(&g_gae_nonfinite_epoch, epoch);
        __hip_atomic_store(&ws.slot[c].w[threadIdx.x], tagged(v, epoch, c, threadIdx.x), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x < kWave) {
        Pair carry = identity_pair();
        bool gave_up = false;
        int width = kFirstBatch;
        for (int64_t j0 = c + 1; j0 < nc; j0 += width, width = kWave) {
            const int64_t k = j0 + lane;
            const bool in = k < nc && lane < width;
            Pair r = identity_pair();
            bool ready = !in;
            int first = kWave;
            for (int poll = 0;; ++poll) {
                if (!ready) ready = read_slot(ws.slot, k, epoch, r);
                const bool cut = in && ready && r.adv.p == 0.f && r.ret.p == 0.f;
                const uint64_t stop = __ballot(!ready || cut);
                first = stop ? __builtin_ctzll(stop) : kWave;
                // Settled when every lane up to the first cut is published.
                const uint64_t unready = __ballot(!ready);
                if (!(unready & ((first < kWave) ? ((2ull << first) - 1) : ~0ull))) break;
                if (poll >= max_polls) {
                    gave_up = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            if (gave_up) break;
            carry = compose<false>(carry, wave_fold<false>((in && lane <= first) ? r : identity_pair()));
            if (first < kWave) break;
        }
        if (lane == 0) {
            if (gave_up) atomicMax(&g_gae_nonfinite_epoch, epoch);
            // The sequence ends with A = G = 0, so the carry is the map applied to 0.
            s_carry[0] = carry.adv.q;
            s_carry[1] = carry.ret.q;
        }
    }
    scan_and_write<false>(g, n, vec, c, s_suffix, s_carry, items, valid_bits);
    if (g.lam_doc) write_lambda(g, ws.cnt, static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x,
                                static_cast<int64_t>(gridDim.x) * kThreads);
}

// Workgroups of k_gae_fix (each takes every gridDim.x-th chunk).
constexpr int kFixBlocks = 512;

// Redoes the outputs of a call whose epoch g_gae_nonfinite_epoch holds (a
// non-finite term, or a wait k_gae_scan gave up), from the slots k_gae_scan
// published: it composes with hardness and folds each chunk's carry from the
// chunks to its right up to the first holding a row end (a non-finite value
// crosses document ends and mask holes in the reference's sequential loop).
// Every other call returns at once.
__global__ __launch_bounds__(kThreads) void k_gae_fix(meshy_gae_args g, Workspace ws, int64_t n, int64_t nc,
                                                      bool vec, unsigned long long epoch) {
    if (g_gae_nonfinite_epoch < epoch) return;
    __shared__ Pair s_wave[kThreads / kWave];
    __shared__ float s_carry[2];
    const int lane = threadIdx.x % kWave;
    for (int64_t c = blockIdx.x; c < nc; c += gridDim.x) {
        Pair items[kItems];
        uint32_t valid_bits;
        bool has_row_end;
        thread_maps(g, ws.cnt, c * kChunk, c * kChunk + static_cast<int64_t>(threadIdx.x) * kItems, n, vec, items,
                    valid_bits, has_row_end);
        if (threadIdx.x < kWave) {
            Pair carry = identity_pair();
            for (int64_t j0 = c + 1; j0 < nc; j0 += kWave) {
                const bool in = j0 + lane < nc;
                const Pair r = in ? slot_pair(ws.slot, j0 + lane) : identity_pair();
                const uint64_t cuts = __ballot(in && is_hard(r.adv.p) && is_hard(r.ret.p));
                const int first = cuts ? __builtin_ctzll(cuts) : kWave;
                carry = compose<true>(carry, wave_fold<true>((in && lane <= first) ? r : identity_pair()));
                if (cuts) break;
            }
            if (lane == 0) {
                s_carry[0] = carry.adv.q;
                s_carry[1] = carry.ret.q;
            }
        }
        scan_and_write<true>(g, n, vec, c, s_wave, s_carry, items, valid_bits);
        __syncthreads();  // s_carry is read after the scan's last barrier
    }
}

// ---------------------------------------------------------------- whitening
// Both passes stream adv and mask in groups of 8 elements (two 16-byte loads
// per array when both are 16-byte aligned), kWhitenGroups groups per thread and
// kWhitenBlockElems elements per workgroup per step.  Every load of a step is
// issued before any is used: group indices past the end are clamped to the last
// group and their elements dropped by a select.  Elements after the last whole
// group (all of them when unaligned) go one per thread, grid-strided.
constexpr int kWhitenThreads = 256;
constexpr int kWhitenGroups = 4;
constexpr int64_t kWhitenBlockElems = static_cast<int64_t>(kWhitenThreads) * kWhitenGroups * 8;
constexpr int64_t kWhitenMaxBlocks = 16384;

inline int whiten_blocks(int64_t n) {
    return static_cast<int>(std::min<int64_t>(kWhitenMaxBlocks, std::max<int64_t>(1, ceil_div(n, kWhitenBlockElems))));
}

__device__ __forceinline__ void whiten_load8(const float* p, int64_t g, float (&v)[8]) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p + 8 * g);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 8 * g + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Per workgroup: the fp64 sum, sum of squares and count over mask != 0
// (vapo.py:22-24) -> partial[3 * block ...].
__global__ __launch_bounds__(kWhitenThreads) void k_whiten_partial(const float* __restrict__ adv,
                                                                   const float* __restrict__ mask, int64_t n,
                                                                   bool vec, double* __restrict__ partial) {
    __shared__ double scratch[kWhitenThreads / kWave];
    double s = 0.0, q = 0.0;
    int c = 0;
    auto add = [&](float x, bool on) {
        const double xd = on ? static_cast<double>(x) : 0.0;
        s += xd;
        q = fma(xd, xd, q);
        c += on;
    };
    const int64_t n8 = vec ? n / 8 : 0;
    for (int64_t g0 = static_cast<int64_t>(blockIdx.x) * kWhitenThreads * kWhitenGroups; g0 < n8;
         g0 += static_cast<int64_t>(gridDim.x) * kWhitenThreads * kWhitenGroups) {
        float x[kWhitenGroups][8], m[kWhitenGroups][8];
#pragma unroll
        for (int k = 0; k < kWhitenGroups; ++k) {
            const int64_t g = min(g0 + k * kWhitenThreads + threadIdx.x, n8 - 1);
            whiten_load8(adv, g, x[k]);
            whiten_load8(mask, g, m[k]);
        }
#pragma unroll
        for (int k = 0; k < kWhitenGroups; ++k) {
            const bool ok = g0 + k * kWhitenThreads + threadIdx.x < n8;
#pragma unroll
            for (int e = 0; e < 8; ++e) add(x[k][e], ok && m[k][e] != 0.f);
        }
    }
    for (int64_t i = 8 * n8 + static_cast<int64_t>(blockIdx.x) * kWhitenThreads + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kWhitenThreads) {
        const float x = adv[i];
        const float mk = mask[i];
        add(x, mk != 0.f);
    }
    s = block_sum<kWhitenThreads>(s, scratch);
    q = block_sum<kWhitenThreads>(q, scratch);
    const double cd = block_sum<kWhitenThreads>(static_cast<double>(c), scratch);
    if (threadIdx.x == 0) {
        partial[3 * blockIdx.x + 0] = s;
        partial[3 * blockIdx.x + 1] = q;
        partial[3 * blockIdx.x + 2] = cd;
    }
}

// The partials folded in a fixed order (bitwise reproducible), divided by the
// replication of the data across ranks (vapo.py:27-28).
__global__ __launch_bounds__(kWhitenThreads) void k_whiten_final(const double* __restrict__ partial, int nb,
                                                                 double replication, double* __restrict__ stats) {
    __shared__ double scratch[kWhitenThreads / kWave];
    constexpr int kIn = 4;  // partials per thread per step, loaded together
    double v[3] = {0.0, 0.0, 0.0};
    for (int b0 = 0; b0 < nb; b0 += kIn * kWhitenThreads) {
        double r[kIn][3];
#pragma unroll
        for (int u = 0; u < kIn; ++u) {
            const int b = min(b0 + u * kWhitenThreads + static_cast<int>(threadIdx.x), nb - 1);
#pragma unroll
            for (int k = 0; k < 3; ++k) r[u][k] = partial[3 * b + k];
        }
#pragma unroll
        for (int u = 0; u < kIn; ++u) {
            const bool ok = b0 + u * kWhitenThreads + static_cast<int>(threadIdx.x) < nb;
#pragma unroll
            for (int k = 0; k < 3; ++k) v[k] += ok ? r[u][k] : 0.0;
        }
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] = block_sum<kWhitenThreads>(v[k], scratch);
    if (threadIdx.x == 0) {
        stats[0] = v[0] / replication;
        stats[1] = v[1] / replication;
        stats[2] = v[2] / replication;
    }
}

// adv <- (adv - mean) * rsqrt(var + 1e-8) where mask != 0, else 0 (vapo.py:25-32):
// the mean, the clamped variance and the Bessel factor when count >= 2.
__global__ __launch_bounds__(kWhitenThreads) void k_whiten_apply(float* __restrict__ adv,
                                                                 const float* __restrict__ mask, int64_t n, bool vec,
                                                                 const double* __restrict__ stats) {
    const double total = stats[0], squares = stats[1], count = stats[2];
    const double cnt = fmax(count, 1.0);
    const double mean = total / cnt;
    double var = fmax(squares / cnt - mean * mean, 0.0);
    if (count >= 2.0) var *= count / (count - 1.0);
    const float mean_f = static_cast<float>(mean);
    const float scale = rsqrtf(static_cast<float>(var) + 1e-8f);
    auto w = [&](float x, float mk) { return (mk != 0.f) ? (x - mean_f) * scale : 0.f; };
    const int64_t n8 = vec ? n / 8 : 0;
    for (int64_t g0 = static_cast<int64_t>(blockIdx.x) * kWhitenThreads * kWhitenGroups; g0 < n8;
         g0 += static_cast<int64_t>(gridDim.x) * kWhitenThreads * kWhitenGroups) {
        float x[kWhitenGroups][8], m[kWhitenGroups][8];
#pragma unroll
        for (int k = 0; k < kWhitenGroups; ++k) {
            const int64_t g = min(g0 + k * kWhitenThreads + threadIdx.x, n8 - 1);
            whiten_load8(adv, g, x[k]);
            whiten_load8(mask, g, m[k]);
        }
#pragma unroll
        for (int k = 0; k < kWhitenGroups; ++k) {
            const int64_t g = g0 + k * kWhitenThreads + threadIdx.x;
            if (g < n8) {
                *reinterpret_cast<f32x4*>(adv + 8 * g) =
                    f32x4{w(x[k][0], m[k][0]), w(x[k][1], m[k][1]), w(x[k][2], m[k][2]), w(x[k][3], m[k][3])};
                *reinterpret_cast<f32x4*>(adv + 8 * g + 4) =
                    f32x4{w(x[k][4], m[k][4]), w(x[k][5], m[k][5]), w(x[k][6], m[k][6]), w(x[k][7], m[k][7])};
            }
        }
    }
    for (int64_t i = 8 * n8 + static_cast<int64_t>(blockIdx.x) * kWhitenThreads + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kWhitenThreads) {
        const float x = adv[i];
        const float mk = mask[i];
        adv[i] = w(x, mk);
    }
}

}  // namespace
}  // namespace meshy

extern "C" size_t meshy_gae_workspace_size(int64_t rows, int64_t S, int64_t n_docs) {
    if (rows < 0 || S < 0 || n_docs < 0) return 0;
    return meshy::ws_bytes(rows * S, n_docs);
}

namespace meshy {
namespace {

// The calls' epochs for g_gae_nonfinite_epoch (process-wide; only growth matters).
std::atomic<unsigned long long> g_gae_epoch{0};
// Polls before k_gae_scan gives a wait up (meshy_gae_set_poll_limit).
std::atomic<int> g_gae_max_polls{kMaxPolls};

int gae_launch(const meshy_gae_args& g, hipStream_t stream) {
    if (g.rows < 0 || g.S < 0 || g.n_docs < 0) return set_error(MESHY_EINVAL, "meshy_gae: negative sizes");
    if (!(g.gamma >= 0.f)) return set_error(MESHY_EINVAL, "meshy_gae: gamma must be non-negative");
    const int64_t n = g.rows * g.S;
    // Without tokens the per-token arrays may be NULL (an empty tensor has no
    // storage); lambda per document is still written.
    if (n > 0 && (!g.rewards || !g.mask || !g.doc_ids))
        return set_error(MESHY_ENULL, "meshy_gae: rewards, mask and doc_ids are required");
    if (n > 0 && g.adv && !g.values) return set_error(MESHY_ENULL, "meshy_gae: advantages need values");
    if (!(g.alpha > 0.f)) return set_error(MESHY_EINVAL, "meshy_gae: alpha must be positive");
    if (!g.workspace || g.workspace_bytes < ws_bytes(n, g.n_docs))
        return set_error(MESHY_ESPACE, "meshy_gae: workspace needs %zu bytes", ws_bytes(n, g.n_docs));
    const int64_t nc = n_chunks_of(n);
    if (nc > INT32_MAX) return set_error(MESHY_EINVAL, "meshy_gae: too many tokens");
    if (g.n_docs > INT32_MAX) return set_error(MESHY_EINVAL, "meshy_gae: too many documents");
    const Workspace ws = ws_of(g.workspace, n, g.n_docs);
    int rc;
    // Document lengths only matter for lambda (advantages / lam_doc), not for returns.
    if (!g.lengths && (g.adv || g.lam_doc) && g.seg_offsets) {
        if (g.n_docs > 0) {
            hipLaunchKernelGGL(k_gae_doc_count, dim3(static_cast<unsigned>(g.n_docs)), dim3(kCountThreads), 0,
                               stream, g.mask, g.seg_offsets, ws.cnt);
            if ((rc = check_launch("meshy_gae(count)"))) return rc;
        }
    } else if (!g.lengths && (g.adv || g.lam_doc)) {
        const int64_t nz = g.n_docs + 1;
        hipLaunchKernelGGL(k_gae_zero, dim3(static_cast<unsigned>(ceil_div(nz, kThreads))), dim3(kThreads), 0, stream,
                           ws.cnt, nz);
        if ((rc = check_launch("meshy_gae(zero)"))) return rc;
        if (n > 0) {
            const int64_t per = static_cast<int64_t>(kCountThreads) * kCountItems;
            hipLaunchKernelGGL(k_gae_count, dim3(static_cast<unsigned>(ceil_div(n, per))), dim3(kCountThreads), 0,
                               stream, g, ws.cnt, n);
            if ((rc = check_launch("meshy_gae(count)"))) return rc;
        }
    }
    // 16-byte vector loads and stores need every per-token array 16-byte aligned
    // (each thread's first position is a multiple of kItems).
    auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool vec = al16(g.rewards) && al16(g.mask) && al16(g.doc_ids) && (!g.values || al16(g.values)) &&
                     (!g.adv || al16(g.adv)) && (!g.returns || al16(g.returns));
    if (nc > 0 && (g.adv || g.returns)) {
        const unsigned long long epoch = g_gae_epoch.fetch_add(1, std::memory_order_relaxed) + 1;
        hipLaunchKernelGGL(k_gae_scan, dim3(static_cast<unsigned>(nc)), dim3(kThreads), 0, stream, g, ws, n, nc, vec,
                           epoch, g_gae_max_polls.load(std::memory_order_relaxed));
        if ((rc = check_launch("meshy_gae(scan)"))) return rc;
        hipLaunchKernelGGL(k_gae_fix, dim3(static_cast<unsigned>(std::min<int64_t>(nc, kFixBlocks))), dim3(kThreads), 0,
                           stream, g, ws, n, nc, vec, epoch);
        if ((rc = check_launch("meshy_gae(fix)"))) return rc;
    } else if (g.lam_doc && g.n_docs > 0) {
        const unsigned nb = static_cast<unsigned>(std::min<int64_t>(1024, ceil_div(g.n_docs, kThreads)));
        hipLaunchKernelGGL(k_gae_lambda, dim3(nb), dim3(kThreads), 0, stream, g, ws.cnt);
        if ((rc = check_launch("meshy_gae(lambda)"))) return rc;
    }
    return MESHY_OK;
}

}  // namespace
}  // namespace meshy

extern "C" int meshy_gae(const meshy_gae_args* args, hipStream_t stream) {
    meshy::clear_error();
    if (!args) return meshy::set_error(MESHY_ENULL, "meshy_gae: args is NULL");
    return meshy::gae_launch(*args, stream);
}

extern "C" int meshy_gae_set_poll_limit(int limit) {
    if (limit < 0) limit = meshy::kMaxPolls;
    return meshy::g_gae_max_polls.exchange(limit);
}

// ------------------------------------------------- _attach_gae_advantages
namespace meshy {
namespace {

constexpr int kAttachThreads = 256;
// Workgroups per sample in k_attach_prep: sample lengths spread over three
// orders of magnitude, and one workgroup per sample leaves the longest one
// bound by a single workgroup's share of a CU.
constexpr int kPrepSplits = 8;

// Token range of split s of a sample [lo, hi): consecutive, each a multiple of 8 long.
__device__ __forceinline__ void split_range(int64_t lo, int64_t hi, int s, int64_t& a, int64_t& b) {
    const int64_t per = ((hi - lo + kPrepSplits - 1) / kPrepSplits + 7) / 8 * 8;
    a = min(lo + per * s, hi);
    b = min(a + per, hi);
}

struct AttachWs {
    float* grid_mask;  // [total] (when the caller passes none)
    float* rewards;    // [total]
    int64_t* doc_ids;  // [total]
    float* lengths;    // [n]
    float* lam;        // [n] (when the caller passes none)
    float* sums;       // [n][4]: sum v*m, sum a*m, sum |a|*m, sum m
    void* gae_ws;
    size_t gae_ws_bytes;
};

size_t attach_ws_bytes(int64_t n, int64_t total) {
    return 3 * align_up(sizeof(float) * total, 256) + align_up(sizeof(int64_t) * total, 256) +
           2 * align_up(sizeof(float) * std::max<int64_t>(n, 1), 256) +
           align_up(sizeof(float) * 4 * std::max<int64_t>(n, 1), 256) + ws_bytes(total, n);
}

AttachWs attach_ws_of(void* base, int64_t n, int64_t total) {
    char* p = static_cast<char*>(base);
    AttachWs w;
    w.grid_mask = reinterpret_cast<float*>(p);
    p += align_up(sizeof(float) * total, 256);
    w.rewards = reinterpret_cast<float*>(p);
    p += align_up(sizeof(float) * total, 256);
    p += align_up(sizeof(float) * total, 256);  // reserved
    w.doc_ids = reinterpret_cast<int64_t*>(p);
    p += align_up(sizeof(int64_t) * total, 256);
    w.lengths = reinterpret_cast<float*>(p);
    p += align_up(sizeof(float) * std::max<int64_t>(n, 1), 256);
    w.lam = reinterpret_cast<float*>(p);
    p += align_up(sizeof(float) * std::max<int64_t>(n, 1), 256);
    w.sums = reinterpret_cast<float*>(p);
    p += align_up(sizeof(float) * 4 * std::max<int64_t>(n, 1), 256);
    w.gae_ws = p;
    w.gae_ws_bytes = ws_bytes(total, n);
    return w;
}

// One workgroup per sample: the next-token grid of trainer.py:656-667.
// The last masked token is found from the sample's end backwards, kLastChunk
// tokens per step (usually one step: the response ends the sample).  The grid
// mask (the mask shifted by one), the reward column and the sample ids are then
// written in wave tiles of 256 tokens; the head and tail one by one.
constexpr int kLastChunk = 4 * kAttachThreads;
constexpr int64_t kWaveTile = 4 * kWave;  // tokens per wave step of k_attach_prep

// mask_assistant as fp32, or as bytes holding 0 or 1 (mask_u8): the same
// values either way.
__device__ __forceinline__ float mask_at(const float* m, int64_t i) { return m[i]; }
__device__ __forceinline__ float mask_at(const uint8_t* m, int64_t i) { return static_cast<float>(m[i]); }
// Tokens i .. i + 3 (i a multiple of 4, the array 16-byte aligned for fp32, 4-byte for bytes).
__device__ __forceinline__ f32x4 mask4(const float* m, int64_t i) { return *reinterpret_cast<const f32x4*>(m + i); }
__device__ __forceinline__ f32x4 mask4(const uint8_t* m, int64_t i) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(m + i);
    return f32x4{static_cast<float>(w & 0xffu), static_cast<float>((w >> 8) & 0xffu),
                 static_cast<float>((w >> 16) & 0xffu), static_cast<float>(w >> 24)};
}

template <typename M>
__global__ __launch_bounds__(kAttachThreads) void k_attach_prep(meshy_gae_attach_args g, AttachWs ws,
                                                                float* grid_mask, float length_const, bool vec) {
    __shared__ int64_t s_last[kAttachThreads / kWave];
    const int64_t j = blockIdx.x;
    const int64_t lo = g.offsets[j];
    const int64_t hi = g.offsets[j + 1];
    const M* m = static_cast<const M*>(g.mask_assistant);
    // Every split finds the sample's last masked position (usually one step).
    int64_t last = -1;  // last masked position, relative to lo
    for (int64_t end = hi; end > lo; end -= kLastChunk) {
        // The four loads take indices clamped into the sample (lo < end) and
        // are all issued before the compares: a load under a per-lane
        // condition compiles to a branch that waits for it.
        float mv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            mv[k] = mask_at(m, max(end - 1 - threadIdx.x - static_cast<int64_t>(k) * kAttachThreads, lo));
        int64_t cand = -1;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t q = end - 1 - threadIdx.x - static_cast<int64_t>(k) * kAttachThreads;
            cand = (q >= lo && mv[k] > 0.f) ? max(cand, q) : cand;
        }
        cand = wave_max(cand);
        if (threadIdx.x % kWave == 0) s_last[threadIdx.x / kWave] = cand;
        __syncthreads();
        cand = s_last[0];
#pragma unroll
        for (int w = 1; w < kAttachThreads / kWave; ++w) cand = max(cand, s_last[w]);
        __syncthreads();
        if (cand >= 0) {
            last = cand - lo;
            break;
        }
    }
    const float r = g.reward[j];
    const int64_t rpos = (last > 0) ? lo + last - 1 : -1;  // where the reward goes
    // Token i of the grid: mask[i + 1] inside the sample, 0 at its last token.
    auto grid_at = [&](int64_t i) { return (i + 1 < hi) ? mask_at(m, i + 1) : 0.f; };
    int64_t a, b;  // this split's tokens
    split_range(lo, hi, static_cast<int>(blockIdx.y), a, b);
    // Wave tiles of 256 tokens from the first multiple of 4: lane l reads and
    // writes tokens [base + 4l, base + 4l + 4) with 16-byte accesses that are
    // contiguous across the wave (whole cache lines per instruction), the
    // ids as two 1 KB halves of 2 tokens per lane.
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
    const int64_t body0 = vec ? min((a + 3) / 4 * 4, b) : b;
    const int64_t n_tiles = (b - body0) / kWaveTile;
    const int64_t body1 = body0 + kWaveTile * n_tiles;
    for (int64_t tile = wid; tile < n_tiles; tile += kAttachThreads / kWave) {
        const int64_t base = body0 + kWaveTile * tile;
        const int64_t i = base + 4 * lane;
        const f32x4 mk = mask4(m, i);
        // mask[i + 4], which lane 63 needs, loaded by every lane with the tile
        // (the other lanes' addresses fall in lines the tile reads anyway).
        const float after = mask_at(m, min(i + 4, hi - 1));
        const float next_lane = __shfl_down(mk.x, 1, kWave);  // mask[i + 4] for lanes 0..62
        const float nx = (lane == kWave - 1) ? (i + 4 < hi ? after : 0.f) : next_lane;
        *reinterpret_cast<f32x4*>(grid_mask + i) = f32x4{mk.y, mk.z, mk.w, nx};
        f32x4 rw{0.f, 0.f, 0.f, 0.f};
        if (rpos >= i && rpos < i + 4) rw[static_cast<int>(rpos - i)] = r;
        *reinterpret_cast<f32x4*>(ws.rewards + i) = rw;
        *reinterpret_cast<i64x2*>(ws.doc_ids + base + 2 * lane) = i64x2{j, j};
        *reinterpret_cast<i64x2*>(ws.doc_ids + base + kWaveTile / 2 + 2 * lane) = i64x2{j, j};
    }
    auto one = [&](int64_t i) {
        grid_mask[i] = grid_at(i);
        ws.rewards[i] = (i == rpos) ? r : 0.f;
        ws.doc_ids[i] = j;
    };
    for (int64_t i = a + threadIdx.x; i < body0; i += kAttachThreads) one(i);
    for (int64_t i = body1 + threadIdx.x; i < b; i += kAttachThreads) one(i);
    if (threadIdx.x == 0 && blockIdx.y == 0) ws.lengths[j] = length_const;
}

// One workgroup per sample: the four sums behind the critic/* metrics.  The
// sample's tokens from the first multiple of 8 are read 8 at a time (16-byte
// loads, four groups of 8 per thread in flight); the head and tail one by one.
struct AttachSums {
    float vm = 0.f, am = 0.f, aam = 0.f, mm = 0.f;
    __device__ void add(float mk, float v, float a) {
        vm = fmaf(v, mk, vm);
        am = fmaf(a, mk, am);
        aam = fmaf(fabsf(a), mk, aam);
        mm += mk;
    }
};

__global__ __launch_bounds__(kAttachThreads) void k_attach_sums(meshy_gae_attach_args g, AttachWs ws,
                                                                const float* grid_mask, bool vec) {
    __shared__ float scratch[kAttachThreads / kWave];
    const int64_t j = blockIdx.x;
    const int64_t lo = g.offsets[j];
    const int64_t hi = g.offsets[j + 1];
    const int64_t body0 = vec ? min((lo + 7) / 8 * 8, hi) : hi;
    const int64_t n8 = (hi - body0) / 8;
    const int64_t body1 = body0 + 8 * n8;
    const uint16_t* vb = static_cast<const uint16_t*>(g.values);
    const float* vf = static_cast<const float*>(g.values);
    AttachSums s[4];
    auto acc8 = [&](int64_t i, AttachSums& a) {
        const f32x4 m0 = *reinterpret_cast<const f32x4*>(grid_mask + i);
        const f32x4 m1 = *reinterpret_cast<const f32x4*>(grid_mask + i + 4);
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(g.adv + i);
        const f32x4 a1 = *reinterpret_cast<const f32x4*>(g.adv + i + 4);
        f32x4 v0, v1;
        if (g.values_bf16) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(vb + i);
            v0 = f32x4{bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y)};
            v1 = f32x4{bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
        } else {
            v0 = *reinterpret_cast<const f32x4*>(vf + i);
            v1 = *reinterpret_cast<const f32x4*>(vf + i + 4);
        }
        a.add(m0.x, v0.x, a0.x); a.add(m0.y, v0.y, a0.y); a.add(m0.z, v0.z, a0.z); a.add(m0.w, v0.w, a0.w);
        a.add(m1.x, v1.x, a1.x); a.add(m1.y, v1.y, a1.y); a.add(m1.z, v1.z, a1.z); a.add(m1.w, v1.w, a1.w);
    };
    auto acc1 = [&](int64_t i) {
        s[1].add(grid_mask[i], g.values_bf16 ? bf16_to_f32(vb[i]) : vf[i], g.adv[i]);
    };
    int64_t c = threadIdx.x;
    for (; c + 3 * kAttachThreads < n8; c += 4 * kAttachThreads) {
        acc8(body0 + 8 * c, s[0]);
        acc8(body0 + 8 * (c + kAttachThreads), s[1]);
        acc8(body0 + 8 * (c + 2 * kAttachThreads), s[2]);
        acc8(body0 + 8 * (c + 3 * kAttachThreads), s[3]);
    }
    for (; c < n8; c += kAttachThreads) acc8(body0 + 8 * c, s[0]);
    for (int64_t i = lo + threadIdx.x; i < body0; i += kAttachThreads) acc1(i);
    for (int64_t i = body1 + threadIdx.x; i < hi; i += kAttachThreads) acc1(i);
    const float vm = block_sum<kAttachThreads>((s[0].vm + s[1].vm) + (s[2].vm + s[3].vm), scratch);
    const float am = block_sum<kAttachThreads>((s[0].am + s[1].am) + (s[2].am + s[3].am), scratch);
    const float aam = block_sum<kAttachThreads>((s[0].aam + s[1].aam) + (s[2].aam + s[3].aam), scratch);
    const float mm = block_sum<kAttachThreads>((s[0].mm + s[1].mm) + (s[2].mm + s[3].mm), scratch);
    if (threadIdx.x == 0) {
        ws.sums[4 * j + 0] = vm;
        ws.sums[4 * j + 1] = am;
        ws.sums[4 * j + 2] = aam;
        ws.sums[4 * j + 3] = mm;
    }
}

__global__ __launch_bounds__(1024) void k_attach_final(meshy_gae_attach_args g, AttachWs ws, const float* lam) {
    __shared__ double s_red[1024 / kWave][6];
    double v[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};  // vm, am, aam, m, per-sequence mean, lambda
    for (int64_t j = threadIdx.x; j < g.n; j += 1024) {
        const float* s = ws.sums + 4 * j;
        v[0] += s[0];
        v[1] += s[1];
        v[2] += s[2];
        v[3] += s[3];
        v[4] += s[1] / fmaxf(s[3], 1.f);
        v[5] += lam[j];
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) v[k] = wave_sum(v[k]);
    if (threadIdx.x % kWave == 0) {
#pragma unroll
        for (int k = 0; k < 6; ++k) s_red[threadIdx.x / kWave][k] = v[k];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double t[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
        for (int w = 0; w < 1024 / kWave; ++w)
#pragma unroll
            for (int k = 0; k < 6; ++k) t[k] += s_red[w][k];
        const double n_tok = fmax(1.0, t[3]);
        const double rows = fmax(1.0, static_cast<double>(g.n));
        g.metrics[0] = static_cast<float>(t[0] / n_tok);
        g.metrics[1] = static_cast<float>(t[1] / n_tok);
        g.metrics[2] = static_cast<float>(t[2] / n_tok);
        g.metrics[3] = static_cast<float>(t[4] / rows);
        g.metrics[4] = static_cast<float>(t[5] / rows);
    }
}

}  // namespace
}  // namespace meshy

extern "C" size_t meshy_gae_attach_workspace_size(int64_t n, int64_t total) {
    if (n < 0 || total < 0) return 0;
    return meshy::attach_ws_bytes(n, total);
}

extern "C" int meshy_gae_attach(const meshy_gae_attach_args* args, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (!args) return set_error(MESHY_ENULL, "meshy_gae_attach: args is NULL");
    const meshy_gae_attach_args& g = *args;
    if (g.n < 0 || g.total < 0) return set_error(MESHY_EINVAL, "meshy_gae_attach: negative sizes");
    if (g.n == 0) return MESHY_OK;
    if (!g.mask_assistant || !g.values || !g.reward || !g.offsets || !g.adv)
        return set_error(MESHY_ENULL, "meshy_gae_attach: mask_assistant, values, reward, offsets and adv are required");
    if (!(g.alpha > 0.f)) return set_error(MESHY_EINVAL, "meshy_gae_attach: alpha must be positive");
    if (g.lambda > 1.f) return set_error(MESHY_EINVAL, "meshy_gae_attach: lambda must be within [0, 1]");
    if (!g.workspace || g.workspace_bytes < attach_ws_bytes(g.n, g.total))
        return set_error(MESHY_ESPACE, "meshy_gae_attach: workspace needs %zu bytes", attach_ws_bytes(g.n, g.total));
    if (g.n > INT32_MAX) return set_error(MESHY_EINVAL, "meshy_gae_attach: too many samples");
    const AttachWs ws = attach_ws_of(g.workspace, g.n, g.total);
    float* grid_mask = g.grid_mask ? g.grid_mask : ws.grid_mask;
    float* lam = g.lam_doc ? g.lam_doc : ws.lam;
    const bool vapo = g.lambda < 0.f;
    // The constant-lambda rule (trainer.py:676-679): lengths chosen so that
    // 1 - 1/(1 * L) == lambda.
    const float length_const =
        vapo ? 0.f : static_cast<float>(1.0 / std::max(1e-9, 1.0 - static_cast<double>(g.lambda)));
    auto al16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    // The wave tiles read the mask 4 tokens at a time: 16 bytes of fp32 or 4 bytes.
    const bool mask_al = reinterpret_cast<uintptr_t>(g.mask_assistant) % (g.mask_u8 ? 4 : 16) == 0;
    const bool vec_prep = mask_al && al16(grid_mask) && al16(ws.rewards) && al16(ws.doc_ids);
    if (g.mask_u8)
        hipLaunchKernelGGL(k_attach_prep<uint8_t>, dim3(static_cast<unsigned>(g.n), kPrepSplits), dim3(kAttachThreads),
                           0, stream, g, ws, grid_mask, length_const, vec_prep);
    else
        hipLaunchKernelGGL(k_attach_prep<float>, dim3(static_cast<unsigned>(g.n), kPrepSplits), dim3(kAttachThreads),
                           0, stream, g, ws, grid_mask, length_const, vec_prep);
    int rc = check_launch("meshy_gae_attach(prep)");
    if (rc) return rc;
    meshy_gae_args a{};
    a.rewards = ws.rewards;
    a.values = g.values;
    a.mask = grid_mask;
    a.doc_ids = ws.doc_ids;
    a.lengths = vapo ? nullptr : ws.lengths;
    a.rows = 1;
    a.S = g.total;
    a.n_docs = g.n;
    a.gamma = g.gamma;
    a.alpha = vapo ? g.alpha : 1.f;
    a.epsilon = g.epsilon;
    a.values_bf16 = g.values_bf16;
    a.adv = g.adv;
    a.returns = nullptr;
    a.lam_doc = lam;
    a.workspace = ws.gae_ws;
    a.workspace_bytes = ws.gae_ws_bytes;
    // Sample j's ids fill [offsets[j], offsets[j+1]): the offsets are the
    // segment offsets of the ids the prep writes.
    a.seg_offsets = g.offsets;
    rc = gae_launch(a, stream);
    if (rc) return rc;
    if (g.metrics) {
        auto al16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
        const bool vec = al16(grid_mask) && al16(g.adv) && al16(g.values);
        hipLaunchKernelGGL(k_attach_sums, dim3(static_cast<unsigned>(g.n)), dim3(kAttachThreads), 0, stream, g, ws,
                           grid_mask, vec);
        if ((rc = check_launch("meshy_gae_attach(sums)"))) return rc;
        hipLaunchKernelGGL(k_attach_final, dim3(1), dim3(1024), 0, stream, g, ws, lam);
        if ((rc = check_launch("meshy_gae_attach(final)"))) return rc;
    }
    return MESHY_OK;
}

extern "C" size_t meshy_whiten_workspace_size(int64_t n) {
    if (n < 0) return 0;
    return sizeof(double) * 3 * static_cast<size_t>(meshy::whiten_blocks(n));
}

extern "C" int meshy_whiten_stats(const float* adv, const float* mask, int64_t n, double replication, double* stats,
                                  void* workspace, size_t workspace_bytes, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (n < 0) return set_error(MESHY_EINVAL, "meshy_whiten_stats: negative size");
    if (!stats || !workspace || (n > 0 && (!adv || !mask)))
        return set_error(MESHY_ENULL, "meshy_whiten_stats: NULL pointer");
    if (workspace_bytes < meshy_whiten_workspace_size(n))
        return set_error(MESHY_ESPACE, "meshy_whiten_stats: workspace needs %zu bytes", meshy_whiten_workspace_size(n));
    if (!(replication > 0.0)) return set_error(MESHY_EINVAL, "meshy_whiten_stats: replication must be positive");
    const int nb = whiten_blocks(n);
    auto al16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    const bool vec = al16(adv) && al16(mask);
    double* partial = static_cast<double*>(workspace);
    hipLaunchKernelGGL(k_whiten_partial, dim3(nb), dim3(kWhitenThreads), 0, stream, adv, mask, n, vec, partial);
    int rc = check_launch("meshy_whiten_stats(partial)");
    if (rc) return rc;
    hipLaunchKernelGGL(k_whiten_final, dim3(1), dim3(kWhitenThreads), 0, stream, partial, nb, replication, stats);
    return check_launch("meshy_whiten_stats(final)");
}

extern "C" int meshy_whiten_apply(float* adv, const float* mask, int64_t n, const double* stats, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (n < 0) return set_error(MESHY_EINVAL, "meshy_whiten_apply: negative size");
    if (n == 0) return MESHY_OK;
    if (!adv || !mask || !stats) return set_error(MESHY_ENULL, "meshy_whiten_apply: NULL pointer");
    auto al16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    const bool vec = al16(adv) && al16(mask);
    hipLaunchKernelGGL(k_whiten_apply, dim3(whiten_blocks(n)), dim3(kWhitenThreads), 0, stream, adv, mask, n, vec,
                       stats);
    return check_launch("meshy_whiten_apply");
}
