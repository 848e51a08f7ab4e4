// mt_device.h -- hand-written gfx950 (CDNA4) device library.
//
// Prepended to every kernel the fragment compiler generates, then compiled
// by hiprtc.  Generated code composes these pieces; the fused elementwise
// expressions arrive as lambdas (prologue transforms, epilogues, merges).
//
//   * mt_dims                 dims passed by value in the kernel arguments
//   * mt_ld4 / mt_st4         128-bit global loads / stores (_nt: nontemporal;
//                             mt_st4_wt: device scope, written through L2)
//   * mt_div_fast             division feeding a matmul (refined reciprocal
//                             times x, within 2 ulp; IEEE division at the edges)
//   * mt_wave_*               wave64 butterfly reductions (fixed order)
//   * mt_tile_colvec / rowvec / scalar
//                             cooperative ROWS x COLS tile fetch: global ->
//                             registers (transform applied to in-bounds
//                             elements, 0 outside), then registers -> LDS;
//                             fetch_raw + commit_xf apply the transform at
//                             commit time instead, so the global loads stay
//                             in flight across the MFMAs of the current chunk
//   * mt_tile_*_g             the same loaders with fetch_gather/commit_apply:
//                             a prologue's full-size operands are loaded with
//                             the tile, the chain is applied at commit
//   * MT_GLOBAL               global address space qualifier (pointer tables
//                             of batched kernels hold global pointers, which
//                             keeps their loads global_load, not flat_load)
//   * mt_tile_dma / mt_swz    direct-to-LDS tile loads (global_load_lds_dwordx4,
//                             no registers, no LDS stores) into dense tiles
//                             whose 16-byte slots are XOR-swizzled per row
//   * mt_mfma_tile            fp32 MFMA (v_mfma_f32_32x32x2f32) over one LDS
//                             k-chunk for a wave's WM x WN grid of 32x32 blocks
//   * mt_mfma_tile_held       the same with the chunk's last group of 4 k-steps
//                             carried over the barrier (mt_mfma_group)
//   * mt_rw_*                 row-owning waves for matmuls 128 columns wide
//                             (16x16x4 MFMAs, A in registers, B in LDS)
//   * mt_acc_row              row of accumulator register v in a 32x32 block
//   * mt_stream_k / mt_sk_*   stream-K schedule of a persistent matmul and the
//                             workspace flags that hand split tiles' partial
//                             sums to the workgroup finishing them
//   * mt_wave_row_reduce / mt_rr_*
//                             row reductions of a matmul's output tile in its
//                             epilogue (lane exchanges, then per-tile values
//                             combined by the last workgroup of a row block)
//
// All indices are unsigned 32-bit except global offsets (size_t).

typedef float mt_f32x4 __attribute__((ext_vector_type(4)));
typedef float mt_f32x16 __attribute__((ext_vector_type(16)));

struct mt_dims {
    unsigned int v[16];
};

#define MT_INLINE __device__ __forceinline__
#define MT_GLOBAL __attribute__((address_space(1)))

#ifndef INFINITY
#define INFINITY __builtin_inff()
#endif
#ifndef NAN
#define NAN __builtin_nanf("")
#endif

MT_INLINE mt_f32x4 mt_ld4(const float* p) { return *reinterpret_cast<const mt_f32x4*>(p); }
MT_INLINE void mt_st4(float* p, mt_f32x4 v) { *reinterpret_cast<mt_f32x4*>(p) = v; }
// Streaming variants: nontemporal hint (data used once; do not keep in cache).
MT_INLINE mt_f32x4 mt_ld4_nt(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const mt_f32x4*>(p));
}
MT_INLINE void mt_st4_nt(float* p, mt_f32x4 v) { __builtin_nontemporal_store(v, reinterpret_cast<mt_f32x4*>(p)); }
// 128-bit global store at device scope (sc1): it writes through the XCD's L2
// instead of leaving a dirty line there, which suits outputs written once by
// streaming kernels.  p must point to global memory (never LDS).  A 128-bit
// store reads its data registers after it issues; the compiler cannot see
// this store, so it is followed by two wait states (see mt_buffer_store4).
MT_INLINE void mt_st4_wt(float* p, mt_f32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}

// x / y where the quotient enters a matmul.  r is the hardware reciprocal
// refined by one Newton step, r + r * (1 - y * r); it depends on y only, so
// the compiler computes it once per distinct divisor (a row or column
// broadcast operand gives one per loaded vector), and each element costs:
//   * 1 <= |y| < 2^125: the product x * r -- within 2 ulp of the IEEE
//     quotient; |x * r| <= |x|, so nothing overflows, and zero, infinite
//     and NaN numerators give what the division gives;
//   * 2^-125 < |y| < 1: the product plus one residual (Markstein) correction
//     q + r * (x - q * y) -- within 1 ulp;
//   * anything else (zero, subnormal, huge or non-finite divisors, quotients
//     of 2^125 and beyond on the second path): the IEEE division.
// Measured on the C5 P.V kernel (one division per A element): 296 us with
// the correction on every element, 276 us with the product alone.
// The two pieces that depend on y alone: the refined reciprocal, and whether
// x * r is the whole quotient (mt_div_plain).  A loader whose divisors are
// all plain computes x * mt_div_rcp(y) directly (commit_apply_fast).
MT_INLINE float mt_div_rcp(float y) {
    const float r = __builtin_amdgcn_rcpf(y);
    return __builtin_fmaf(__builtin_fmaf(-y, r, 1.0f), r, r);
}
MT_INLINE bool mt_div_plain(float y) {
    const float ay = __builtin_fabsf(y);
    return ay >= 1.0f && ay < 0x1.0p+125f;
}
MT_INLINE float mt_div_fast(float x, float y) {
    const float ay = __builtin_fabsf(y);
    const float r = mt_div_rcp(y);
    const float q = x * r;
    if (__builtin_expect(mt_div_plain(y), 1)) return q;
    const float v = __builtin_fmaf(__builtin_fmaf(-q, y, x), r, q);
    const bool ok = ay > 0x1.0p-125f && ay < 1.0f && __builtin_fabsf(v) < 0x1.0p+125f;
    // The IEEE division stays on its (rarely taken) branch: the empty asm
    // statement emits nothing but cannot be speculated, so the compiler does
    // not compute the division for every lane and select.
    if (__builtin_expect(!ok, 0)) {
        float xs = x;
        asm volatile("" : "+v"(xs));
        return xs / y;
    }
    return v;
}

MT_INLINE unsigned mt_lane() { return threadIdx.x & 63u; }
// Wave index as a scalar (wave-uniform) value.
MT_INLINE unsigned mt_wave() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ---------------------------------------------------------------------------
// wave64 reductions.  Butterfly over xor offsets 32, 16, 8, 4, 2, 1: after
// step `off`, lane l holds v_l (op) v_{l^off}.  Every lane ends with the same
// value; the pairing tree is fixed, so results are reproducible (and the CPU
// oracle replays the same tree).
// ---------------------------------------------------------------------------

MT_INLINE float mt_shfl_xor(float v, int off) { return __shfl_xor(v, off, 64); }

MT_INLINE float mt_wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = v + mt_shfl_xor(v, off);
    return v;
}
MT_INLINE float mt_wave_product(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = v * mt_shfl_xor(v, off);
    return v;
}
MT_INLINE float mt_wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, mt_shfl_xor(v, off));
    return v;
}
MT_INLINE float mt_wave_min(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fminf(v, mt_shfl_xor(v, off));
    return v;
}

// ---------------------------------------------------------------------------
// Cooperative tile loaders.  A loader owns the registers for its share of one
// ROWS x COLS tile (NT lanes).  fetch<CHECK>() issues the global loads for the
// tile at (row0, col0) of a strided matrix (element (r, c) at
// src[r*rs + c*cs]); F(raw, row, col) transforms each in-bounds element
// (elementwise prologue); elements outside (rlim, clim) are 0 (identity of
// the matmul / sum consumer).  commit<LD>() writes the registers into an LDS
// tile with row pitch LD floats.  Splitting the two lets the mainloop keep
// the next tile's loads in flight while the MFMAs run.
// ---------------------------------------------------------------------------

struct mt_identity {
    MT_INLINE float operator()(float v, unsigned, unsigned) const { return v; }
};

// Partial fetches.  Every fetch takes an optional (q, Q): it then issues only
// the loads of part q of Q, slot i of n belonging to part (i * Q) / n, so Q
// calls with q = 0 .. Q-1 issue every load exactly once (the default 0, 1 is
// the whole tile).  The mainloop spreads a chunk's loads over the MFMA
// sequence this way instead of issuing them in one burst: a burst of vector
// memory instructions holds each wave in load issue while the address units
// work through it, and its MFMAs wait behind them.
__host__ __device__ __forceinline__ constexpr bool mt_in_part(int i, int n, int q, int Q) {
    return Q <= 1 || (i * Q) / n == q;
}

// Vectorised along columns: cs == 1, rs % 4 == 0, COLS % 4 == 0, clim % 4 == 0.
template <int ROWS, int COLS, int NT>
struct mt_tile_colvec {
    static constexpr int CV = COLS / 4;
    static constexpr int TOTAL = ROWS * CV;
    static constexpr int PER = (TOTAL + NT - 1) / NT;
    mt_f32x4 v[PER];

    template <bool CHECK, typename F>
    MT_INLINE void fetch(const float* __restrict__ src, unsigned rs, unsigned row0, unsigned col0,
                         unsigned rlim, unsigned clim, unsigned tid, F f, int q = 0, int Q = 1) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (!mt_in_part(i, PER, q, Q)) continue;
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / CV, c = (idx % CV) * 4u;
            const unsigned gr = row0 + r, gc = col0 + c;
            mt_f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < rlim && gc < clim))) {
                x = mt_ld4(src + (size_t)gr * rs + gc);
                x.x = f(x.x, gr, gc);
                x.y = f(x.y, gr, gc + 1u);
                x.z = f(x.z, gr, gc + 2u);
                x.w = f(x.w, gr, gc + 3u);
            }
            v[i] = x;
        }
    }

    // Any row stride, limits and base alignment (the strides and limits are
    // run-time values): a slot is loaded with one 128-bit load when its row
    // start is 16-byte aligned and all 4 columns are in bounds, otherwise
    // element by element (out-of-bounds elements are 0, and f is applied to
    // in-bounds elements only).  Same register layout as fetch().
    template <typename F>
    MT_INLINE void fetch_safe(const float* __restrict__ src, unsigned rs, unsigned row0, unsigned col0,
                              unsigned rlim, unsigned clim, unsigned tid, F f, int q = 0, int Q = 1) {
        const bool aligned =
            ((rs & 3u) == 0u) && ((reinterpret_cast<unsigned long long>(src) & 15ull) == 0ull) && ((col0 & 3u) == 0u);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (!mt_in_part(i, PER, q, Q)) continue;
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / CV, c = (idx % CV) * 4u;
            const unsigned gr = row0 + r, gc = col0 + c;
            mt_f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && gr < rlim && gc < clim) {
                const float* p = src + (size_t)gr * rs + gc;
                if (aligned && gc + 3u < clim) {
                    x = mt_ld4(p);
                    x.x = f(x.x, gr, gc);
                    x.y = f(x.y, gr, gc + 1u);
                    x.z = f(x.z, gr, gc + 2u);
                    x.w = f(x.w, gr, gc + 3u);
                } else {
                    x.x = f(p[0], gr, gc);
                    if (gc + 1u < clim) x.y = f(p[1], gr, gc + 1u);
                    if (gc + 2u < clim) x.z = f(p[2], gr, gc + 2u);
                    if (gc + 3u < clim) x.w = f(p[3], gr, gc + 3u);
                }
            }
            v[i] = x;
        }
    }

    // 128-bit LDS stores when the row pitch keeps them 16-byte aligned.
    template <int LD>
    MT_INLINE void commit(float* lds, unsigned tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            if (TOTAL % NT == 0 || idx < (unsigned)TOTAL) {
                const unsigned r = idx / CV, c = (idx % CV) * 4u;
                if constexpr (LD % 4 == 0) {
                    mt_st4(lds + r * LD + c, v[i]);
                } else {
                    float* d = lds + r * LD + c;
                    d[0] = v[i].x, d[1] = v[i].y, d[2] = v[i].z, d[3] = v[i].w;
                }
            }
        }
    }

    // Deferred transform: fetch_raw keeps the loaded values untouched (0
    // outside the bounds) and remembers the tile origin; commit_xf applies f
    // to the in-bounds elements on the way to LDS.
    unsigned r0, c0, rl, cl;

    template <bool CHECK>
    MT_INLINE void fetch_raw(const float* __restrict__ src, unsigned rs, unsigned row0, unsigned col0,
                             unsigned rlim, unsigned clim, unsigned tid, int q = 0, int Q = 1) {
        r0 = row0, c0 = col0, rl = rlim, cl = clim;
        fetch<CHECK>(src, rs, row0, col0, rlim, clim, tid, mt_identity{}, q, Q);
    }

    template <int LD, bool CHECK, typename F>
    MT_INLINE void commit_xf(float* lds, unsigned tid, F f) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / CV, c = (idx % CV) * 4u;
            const unsigned gr = r0 + r, gc = c0 + c;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < rl && gc < cl))) {
                v[i].x = f(v[i].x, gr, gc);
                v[i].y = f(v[i].y, gr, gc + 1u);
                v[i].z = f(v[i].z, gr, gc + 2u);
                v[i].w = f(v[i].w, gr, gc + 3u);
            }
        }
        commit<LD>(lds, tid);
    }
};

// Vectorised along rows: rs == 1, cs % 4 == 0, ROWS % 4 == 0, rlim % 4 == 0.
template <int ROWS, int COLS, int NT>
struct mt_tile_rowvec {
    static constexpr int RV = ROWS / 4;
    static constexpr int TOTAL = RV * COLS;
    static constexpr int PER = (TOTAL + NT - 1) / NT;
    mt_f32x4 v[PER];

    template <bool CHECK, typename F>
    MT_INLINE void fetch(const float* __restrict__ src, unsigned cs, unsigned row0, unsigned col0,
                         unsigned rlim, unsigned clim, unsigned tid, F f, int q = 0, int Q = 1) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (!mt_in_part(i, PER, q, Q)) continue;
            const unsigned idx = tid + i * NT;
            const unsigned c = idx / RV, r = (idx % RV) * 4u;
            const unsigned gr = row0 + r, gc = col0 + c;
            mt_f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < rlim && gc < clim))) {
                x = mt_ld4(src + gr + (size_t)gc * cs);
                x.x = f(x.x, gr, gc);
                x.y = f(x.y, gr + 1u, gc);
                x.z = f(x.z, gr + 2u, gc);
                x.w = f(x.w, gr + 3u, gc);
            }
            v[i] = x;
        }
    }

    template <int LD>
    MT_INLINE void commit(float* lds, unsigned tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            if (TOTAL % NT == 0 || idx < (unsigned)TOTAL) {
                const unsigned c = idx / RV, r = (idx % RV) * 4u;
                lds[(r + 0u) * LD + c] = v[i].x;
                lds[(r + 1u) * LD + c] = v[i].y;
                lds[(r + 2u) * LD + c] = v[i].z;
                lds[(r + 3u) * LD + c] = v[i].w;
            }
        }
    }

    unsigned r0, c0, rl, cl;

    template <bool CHECK>
    MT_INLINE void fetch_raw(const float* __restrict__ src, unsigned cs, unsigned row0, unsigned col0,
                             unsigned rlim, unsigned clim, unsigned tid, int q = 0, int Q = 1) {
        r0 = row0, c0 = col0, rl = rlim, cl = clim;
        fetch<CHECK>(src, cs, row0, col0, rlim, clim, tid, mt_identity{}, q, Q);
    }

    template <int LD, bool CHECK, typename F>
    MT_INLINE void commit_xf(float* lds, unsigned tid, F f) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            const unsigned c = idx / RV, r = (idx % RV) * 4u;
            const unsigned gr = r0 + r, gc = c0 + c;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < rl && gc < cl))) {
                v[i].x = f(v[i].x, gr, gc);
                v[i].y = f(v[i].y, gr + 1u, gc);
                v[i].z = f(v[i].z, gr + 2u, gc);
                v[i].w = f(v[i].w, gr + 3u, gc);
            }
        }
        commit<LD>(lds, tid);
    }
};

// Any strides: one element per load.
template <int ROWS, int COLS, int NT>
struct mt_tile_scalar {
    static constexpr int TOTAL = ROWS * COLS;
    static constexpr int PER = (TOTAL + NT - 1) / NT;
    float v[PER];

    template <bool CHECK, typename F>
    MT_INLINE void fetch(const float* __restrict__ src, unsigned rs, unsigned cs, unsigned row0,
                         unsigned col0, unsigned rlim, unsigned clim, unsigned tid, F f, int q = 0, int Q = 1) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (!mt_in_part(i, PER, q, Q)) continue;
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / COLS, c = idx % COLS;
            const unsigned gr = row0 + r, gc = col0 + c;
            float x = 0.f;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < rlim && gc < clim))) {
                x = f(src[(size_t)gr * rs + (size_t)gc * cs], gr, gc);
            }
            v[i] = x;
        }
    }

    template <int LD>
    MT_INLINE void commit(float* lds, unsigned tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            if (TOTAL % NT == 0 || idx < (unsigned)TOTAL) {
                const unsigned r = idx / COLS, c = idx % COLS;
                lds[r * LD + c] = v[i];
            }
        }
    }

    unsigned r0, c0, rl, cl;

    template <bool CHECK>
    MT_INLINE void fetch_raw(const float* __restrict__ src, unsigned rs, unsigned cs, unsigned row0,
                             unsigned col0, unsigned rlim, unsigned clim, unsigned tid, int q = 0, int Q = 1) {
        r0 = row0, c0 = col0, rl = rlim, cl = clim;
        fetch<CHECK>(src, rs, cs, row0, col0, rlim, clim, tid, mt_identity{}, q, Q);
    }

    template <int LD, bool CHECK, typename F>
    MT_INLINE void commit_xf(float* lds, unsigned tid, F f) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / COLS, c = idx % COLS;
            const unsigned gr = r0 + r, gc = c0 + c;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < rl && gc < cl))) {
                v[i] = f(v[i], gr, gc);
            }
        }
        commit<LD>(lds, tid);
    }
};

// ---------------------------------------------------------------------------
// Gather / apply loaders: a prologue that reads E full-size operands loads
// them together with the tile (fetch_gather: g(row, col) -> mt_vals<E> per
// element) and applies the chain when the tile is committed to LDS
// (commit_apply: a(raw, extras) per in-bounds element), so neither the tile
// nor its operands are waited for before the current chunk's MFMAs.  Out of
// bounds elements stay 0 and are not transformed.  SLOT = true (vectorised
// loaders): the operands are constant along the vector axis (a column
// broadcast for mt_tile_colvec_g, a row broadcast for mt_tile_rowvec_g), so
// they are gathered once per 128-bit slot and the 4 elements share them --
// one value, so work that depends only on it (a divisor's reciprocal) is
// done once per slot.
// ---------------------------------------------------------------------------

template <int E>
struct mt_vals {
    float v[E];
};

template <int ROWS, int COLS, int NT, int E, bool SLOT = false>
struct mt_tile_colvec_g : mt_tile_colvec<ROWS, COLS, NT> {
    using Base = mt_tile_colvec<ROWS, COLS, NT>;
    using Base::CV;
    using Base::PER;
    using Base::TOTAL;
    static constexpr int NG = SLOT ? 1 : 4;  // gathers per slot
    mt_vals<E> ex[PER][NG];

    template <bool CHECK, typename G>
    MT_INLINE void fetch_gather(const float* __restrict__ src, unsigned rs, unsigned row0, unsigned col0,
                                unsigned rlim, unsigned clim, unsigned tid, G g, int q = 0, int Q = 1) {
        this->r0 = row0, this->c0 = col0, this->rl = rlim, this->cl = clim;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (!mt_in_part(i, PER, q, Q)) continue;
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / CV, c = (idx % CV) * 4u;
            const unsigned gr = row0 + r, gc = col0 + c;
            mt_f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < rlim && gc < clim))) {
                x = mt_ld4(src + (size_t)gr * rs + gc);
#pragma unroll
                for (int j = 0; j < NG; ++j) ex[i][j] = g(gr, gc + (unsigned)j);
            }
            this->v[i] = x;
        }
    }

    // SLOT gathers are constant along the loaded rows' k axis, so the next
    // chunk of the same tile needs the same operands: fetch_keep loads the
    // tile alone and keeps ex (and the work derived from it, such as a
    // divisor's reciprocal, stays loop-invariant for the compiler).
    template <bool CHECK>
    MT_INLINE void fetch_keep(const float* __restrict__ src, unsigned rs, unsigned row0, unsigned col0,
                              unsigned rlim, unsigned clim, unsigned tid, int q = 0, int Q = 1) {
        static_assert(SLOT, "only per-slot gathers are invariant along k");
        this->r0 = row0, this->c0 = col0, this->rl = rlim, this->cl = clim;
        Base::template fetch<CHECK>(src, rs, row0, col0, rlim, clim, tid, mt_identity{}, q, Q);
    }

    // True in every lane when P(e) holds for the gathered operands of every
    // in-bounds slot of every lane of the wave (one wave-uniform test).
    template <bool CHECK, typename P>
    MT_INLINE bool all_plain(unsigned tid, P p) const {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / CV, c = (idx % CV) * 4u;
            const unsigned gr = this->r0 + r, gc = this->c0 + c;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < this->rl && gc < this->cl))) {
#pragma unroll
                for (int j = 0; j < NG; ++j) ok = ok && p(ex[i][j]);
            }
        }
        return __builtin_amdgcn_ballot_w64(!ok) == 0ull;
    }

    // commit_apply with Q -- the chain with its divisions reduced to
    // x * mt_div_rcp(y), exact when P holds -- when all_plain, without a
    // branch per element; A otherwise.
    template <int LD, bool CHECK, typename A, typename Q, typename P>
    MT_INLINE void commit_apply_fast(float* lds, unsigned tid, A a, Q q, P p) {
        if (__builtin_expect(all_plain<CHECK>(tid, p), 1)) {
            commit_apply<LD, CHECK>(lds, tid, q);
        } else {
            commit_apply<LD, CHECK>(lds, tid, a);
        }
    }

    template <int LD, bool CHECK, typename A>
    MT_INLINE void commit_apply(float* lds, unsigned tid, A a) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / CV, c = (idx % CV) * 4u;
            const unsigned gr = this->r0 + r, gc = this->c0 + c;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < this->rl && gc < this->cl))) {
                this->v[i].x = a(this->v[i].x, ex[i][0]);
                this->v[i].y = a(this->v[i].y, ex[i][1 % NG]);
                this->v[i].z = a(this->v[i].z, ex[i][2 % NG]);
                this->v[i].w = a(this->v[i].w, ex[i][3 % NG]);
            }
        }
        Base::template commit<LD>(lds, tid);
    }
};

template <int ROWS, int COLS, int NT, int E, bool SLOT = false>
struct mt_tile_rowvec_g : mt_tile_rowvec<ROWS, COLS, NT> {
    using Base = mt_tile_rowvec<ROWS, COLS, NT>;
    using Base::RV;
    using Base::PER;
    using Base::TOTAL;
    static constexpr int NG = SLOT ? 1 : 4;  // gathers per slot
    mt_vals<E> ex[PER][NG];

    template <bool CHECK, typename G>
    MT_INLINE void fetch_gather(const float* __restrict__ src, unsigned cs, unsigned row0, unsigned col0,
                                unsigned rlim, unsigned clim, unsigned tid, G g, int q = 0, int Q = 1) {
        this->r0 = row0, this->c0 = col0, this->rl = rlim, this->cl = clim;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (!mt_in_part(i, PER, q, Q)) continue;
            const unsigned idx = tid + i * NT;
            const unsigned c = idx / RV, r = (idx % RV) * 4u;
            const unsigned gr = row0 + r, gc = col0 + c;
            mt_f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < rlim && gc < clim))) {
                x = mt_ld4(src + gr + (size_t)gc * cs);
#pragma unroll
                for (int j = 0; j < NG; ++j) ex[i][j] = g(gr + (unsigned)j, gc);
            }
            this->v[i] = x;
        }
    }

    template <bool CHECK>
    MT_INLINE void fetch_keep(const float* __restrict__ src, unsigned cs, unsigned row0, unsigned col0,
                              unsigned rlim, unsigned clim, unsigned tid, int q = 0, int Q = 1) {
        static_assert(SLOT, "only per-slot gathers are invariant along k");
        this->r0 = row0, this->c0 = col0, this->rl = rlim, this->cl = clim;
        Base::template fetch<CHECK>(src, cs, row0, col0, rlim, clim, tid, mt_identity{}, q, Q);
    }

    // True in every lane when P(e) holds for the gathered operands of every
    // in-bounds slot of every lane of the wave (one wave-uniform test).
    template <bool CHECK, typename P>
    MT_INLINE bool all_plain(unsigned tid, P p) const {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            const unsigned c = idx / RV, r = (idx % RV) * 4u;
            const unsigned gr = this->r0 + r, gc = this->c0 + c;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < this->rl && gc < this->cl))) {
#pragma unroll
                for (int j = 0; j < NG; ++j) ok = ok && p(ex[i][j]);
            }
        }
        return __builtin_amdgcn_ballot_w64(!ok) == 0ull;
    }

    // commit_apply with Q -- the chain with its divisions reduced to
    // x * mt_div_rcp(y), exact when P holds -- when all_plain, without a
    // branch per element; A otherwise.
    template <int LD, bool CHECK, typename A, typename Q, typename P>
    MT_INLINE void commit_apply_fast(float* lds, unsigned tid, A a, Q q, P p) {
        if (__builtin_expect(all_plain<CHECK>(tid, p), 1)) {
            commit_apply<LD, CHECK>(lds, tid, q);
        } else {
            commit_apply<LD, CHECK>(lds, tid, a);
        }
    }

    template <int LD, bool CHECK, typename A>
    MT_INLINE void commit_apply(float* lds, unsigned tid, A a) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            const unsigned c = idx / RV, r = (idx % RV) * 4u;
            const unsigned gr = this->r0 + r, gc = this->c0 + c;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < this->rl && gc < this->cl))) {
                this->v[i].x = a(this->v[i].x, ex[i][0]);
                this->v[i].y = a(this->v[i].y, ex[i][1 % NG]);
                this->v[i].z = a(this->v[i].z, ex[i][2 % NG]);
                this->v[i].w = a(this->v[i].w, ex[i][3 % NG]);
            }
        }
        Base::template commit<LD>(lds, tid);
    }
};

template <int ROWS, int COLS, int NT, int E>
struct mt_tile_scalar_g : mt_tile_scalar<ROWS, COLS, NT> {
    using Base = mt_tile_scalar<ROWS, COLS, NT>;
    using Base::PER;
    using Base::TOTAL;
    mt_vals<E> ex[PER];

    template <bool CHECK, typename G>
    MT_INLINE void fetch_gather(const float* __restrict__ src, unsigned rs, unsigned cs, unsigned row0,
                                unsigned col0, unsigned rlim, unsigned clim, unsigned tid, G g, int q = 0,
                                int Q = 1) {
        this->r0 = row0, this->c0 = col0, this->rl = rlim, this->cl = clim;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (!mt_in_part(i, PER, q, Q)) continue;
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / COLS, c = idx % COLS;
            const unsigned gr = row0 + r, gc = col0 + c;
            float x = 0.f;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < rlim && gc < clim))) {
                x = src[(size_t)gr * rs + (size_t)gc * cs];
                ex[i] = g(gr, gc);
            }
            this->v[i] = x;
        }
    }

    template <int LD, bool CHECK, typename A>
    MT_INLINE void commit_apply(float* lds, unsigned tid, A a) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const unsigned idx = tid + i * NT;
            const unsigned r = idx / COLS, c = idx % COLS;
            const unsigned gr = this->r0 + r, gc = this->c0 + c;
            if ((TOTAL % NT == 0 || idx < (unsigned)TOTAL) && (!CHECK || (gr < this->rl && gc < this->cl))) {
                this->v[i] = a(this->v[i], ex[i]);
            }
        }
        Base::template commit<LD>(lds, tid);
    }
};

// Integer helpers callable from host code too (the CPU tests check them).
#define MT_HD __host__ __device__ __forceinline__

// ---------------------------------------------------------------------------
// Direct-to-LDS tile loads (gfx950 global_load_lds_dwordx4).  One such load
// moves 16 bytes per lane from global memory straight into LDS at
// M0 + 16 * lane, so a wave writes 1 KiB of contiguous LDS per instruction
// and no registers or LDS-store instructions are spent on the tile.  Tiles
// are therefore dense; operand tiles the MFMAs read row-wise with 128-bit
// reads permute the 16-byte slots of each row by mt_swz (an XOR of the
// slot index), which keeps those reads free of bank conflicts.
//
// The loads are issued from inline asm: the compiler then does not see an
// LDS write it would wait for before every later LDS read (it cannot tell
// the stage being filled from the one being read).  The mainloop waits for
// them itself (s_waitcnt) before the barrier that publishes the chunk.
// ---------------------------------------------------------------------------

// Physical slot permutation of row r of a dense LDS tile with S 16-byte slots
// per row (slot p holds logical slot p ^ mt_swz<S>(r)).  It depends on
// r mod 16 only, and makes the slots read by 8 consecutive rows, and by the
// even and the odd rows among 16 consecutive ones, pairwise distinct -- a
// 128-bit read of one slot per row by consecutive lanes then meets no bank
// conflict whether the LDS serves 128 or 256 bytes per cycle.
template <int S>
MT_HD unsigned mt_swz(unsigned r) {
    static_assert(S == 4 || S == 8, "swizzle defined for 16- and 32-float rows");
    if constexpr (S == 8) return ((r >> 1) ^ ((r & 1u) << 2)) & 7u;
    return ((r >> 1) ^ (r >> 2)) & 3u;
}

MT_INLINE unsigned mt_lds_addr(const float* p) {
    return (unsigned)(unsigned long long)(const __attribute__((address_space(3))) float*)p;
}

// 16 bytes from sbase + voff to LDS byte address lds_byte + 16 * lane:
// sbase is a wave-uniform address held in scalar registers, voff this lane's
// 32-bit byte offset from it, lds_byte wave uniform.  One wait state
// separates the M0 write from the load reading it.
MT_INLINE void mt_dma16(unsigned long long sbase, unsigned voff, unsigned lds_byte) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_byte)
                 : "memory", "m0");
}

// A wave-uniform address as a scalar value (both halves read from the first
// lane; the compiler folds this when the address is already scalar).
MT_INLINE unsigned long long mt_uniform_addr(const float* p) {
    const unsigned long long a = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)a);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
    return ((unsigned long long)hi << 32) | lo;
}

// Where a direct-to-LDS load puts its data: lane `lane` of wave-load `inst`
// writes physical slot 64 inst + lane of a dense tile with S slots per row,
// i.e. row r, physical slot p; it loads the row's logical slot p (SWZ: p ^
// mt_swz<S>(r)), so logical slot L of row r sits at physical L ^ mt_swz<S>(r).
template <int S, bool SWZ>
MT_HD void mt_dma_slot(unsigned inst, unsigned lane, unsigned& r, unsigned& logical) {
    const unsigned slot = inst * 64u + lane;
    r = slot / S;
    logical = slot % S;
    if constexpr (SWZ) logical ^= mt_swz<S>(r);
}

// ROWS x COLS tile of a row-major source (row stride rs floats, a multiple of
// 4; 16-byte aligned base) at (row0, col0), every element in bounds, into a
// dense LDS tile; SWZ permutes each row's slots by mt_swz.  Wave w issues
// wave-loads w PERW .. w PERW + PERW - 1, each 1 KiB of contiguous LDS.
//
// The loader is built once per kernel with the source's row stride: each
// lane's byte offsets from the tile origin do not change from chunk to
// chunk, so they are computed there, and a fetch adds only the tile
// origin -- a scalar address -- through the load's scalar-base form.  The
// offsets are 32-bit: ((ROWS - 1) rs + COLS) * 4 must stay below 2^32 (the
// assembler checks).  Recomputing the full per-lane addresses in every
// chunk cost ~900 cycles of VALU work per 32-wide chunk on a 256x256 tile
// (4096^3 GEMM, measured in shader cycles per workgroup: 2.26 -> 2.19 M).
template <int ROWS, int COLS, int NT, bool SWZ>
struct mt_tile_dma {
    static constexpr int S = COLS / 4;
    static constexpr int INSTR = ROWS * S / 64;
    static constexpr int PERW = INSTR / (NT / 64);
    static_assert(COLS % 4 == 0 && (ROWS * S) % 64 == 0 && INSTR % (NT / 64) == 0,
                  "the tile must split into whole 1 KiB wave loads, the same number per wave");
    unsigned off[PERW];  // this lane's byte offset of each of the wave's loads
    unsigned lds_off;    // byte offset of the wave's first load in the tile (uniform)

    MT_INLINE mt_tile_dma(unsigned rs, unsigned tid) {
        const unsigned lane = tid & 63u;
        const unsigned wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        lds_off = wave * PERW * 1024u;
#pragma unroll
        for (int q = 0; q < PERW; ++q) {
            unsigned r, logical;
            mt_dma_slot<S, SWZ>(wave * PERW + q, lane, r, logical);
            off[q] = (r * rs + 4u * logical) * 4u;
        }
    }

    // rs: the row stride the loader was built with.
    MT_INLINE void fetch(const float* __restrict__ src, unsigned rs, unsigned row0, unsigned col0, float* lds,
                         int part = 0, int parts = 1) const {
        const unsigned long long origin = mt_uniform_addr(src + (size_t)row0 * rs + col0);
        const unsigned base = __builtin_amdgcn_readfirstlane(mt_lds_addr(lds)) + lds_off;
#pragma unroll
        for (int q = 0; q < PERW; ++q) {
            if (!mt_in_part(q, PERW, part, parts)) continue;
            mt_dma16(origin, off[q], base + (unsigned)q * 1024u);
        }
    }
};

// ---------------------------------------------------------------------------
// fp32 MFMA over one LDS k-chunk.
//
// v_mfma_f32_32x32x2f32 computes D[32x32] += A[32x2] * B[2x32]; lane l supplies
// A[l%32][l/32] and B[l/32][l%32].  The two k slots of one instruction are
// taken from the two halves of the chunk: lane half h = l/32 feeds chunk
// column k = h*TK/2 + s at step s.  Both operands use the same mapping, so
// every product A[i][k]*B[k][j] of the chunk is accumulated exactly once, and
// consecutive steps s read consecutive A elements (128-bit LDS reads).
//
// As points at the wave's first A row in an LDS tile [rows][LDA] (row-major,
// m x k); Bs at the wave's first column in an LDS tile [TK][LDB] (k x n).
// acc[i][j] is the 32x32 block at rows 32*i, cols 32*j of the wave tile.
//
// Layouts: A rows of LDA floats, or (ASWZ) a dense [rows][TK] tile written by
// direct-to-LDS loads whose 16-byte slots are permuted by mt_swz; B either
// [TK][LDB] (k-major), or (BNM) n-major [cols][TK] swizzled like A and read
// 128 bits at a time.  Every layout feeds the MFMAs the same values in the
// same order, so results are identical across layouts.
// ---------------------------------------------------------------------------

// hook(q) runs at the start of each group of 4 k-steps, q = 0 .. TK/8 - 1:
// the mainloop issues its next chunk's loads there, spread over the MFMAs.
struct mt_no_hook {
    MT_INLINE void operator()(int) const {}
};

template <int WM, int WN, int TK, int LDA, int LDB, bool ASWZ = false, bool BNM = false, typename H = mt_no_hook>
MT_INLINE void mt_mfma_tile(const float* __restrict__ As, const float* __restrict__ Bs,
                            mt_f32x16 (&acc)[WM][WN], unsigned lane, H hook = H{}) {
    static_assert(TK % 8 == 0, "TK must be a multiple of 8");
    static_assert(LDA % 4 == 0, "LDA must keep 16-byte alignment");
    static_assert(!ASWZ || LDA == TK, "a swizzled A tile is dense");
    static_assert(!BNM || LDB == TK, "an n-major B tile is dense");
    constexpr int HALF = TK / 2;
    const unsigned li = lane & 31u;
    const unsigned lh = lane >> 5;
    // Swizzled tiles: the wave's first row is a multiple of 16, so row
    // 32 i + li of the wave permutes its slots by mt_swz(li).
    unsigned m = 0u;
    if constexpr (ASWZ || BNM) m = mt_swz<TK / 4>(li);
    const float* a_base = ASWZ ? As + li * TK : As + li * LDA + lh * HALF;
    const float* b_base = BNM ? Bs + li * TK : Bs + (lh * HALF) * LDB + li;
    // Raise this wave's issue priority while it feeds the matrix core, so a
    // wave still holding MFMAs is preferred over one writing the next chunk
    // to LDS or waiting at the barrier (measured +2.6-3.6 % on 4096^3 and
    // C4 GEMMs).  The priority of instruction issue inside a SIMD only.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s0 = 0; s0 < HALF; s0 += 4) {
        hook(s0 / 4);
        const unsigned slot = (lh * HALF + (unsigned)s0) / 4u;  // swizzled tiles: logical 16-byte slot
        mt_f32x4 a[WM];
#pragma unroll
        for (int i = 0; i < WM; ++i)
            a[i] = ASWZ ? mt_ld4(a_base + i * 32 * TK + 4u * (slot ^ m)) : mt_ld4(a_base + i * 32 * LDA + s0);
        mt_f32x4 bv[BNM ? WN : 1];
        if constexpr (BNM) {
#pragma unroll
            for (int j = 0; j < WN; ++j) bv[j] = mt_ld4(b_base + j * 32 * TK + 4u * (slot ^ m));
        }
#pragma unroll
        for (int ss = 0; ss < 4; ++ss) {
            float b[WN];
#pragma unroll
            for (int j = 0; j < WN; ++j) b[j] = BNM ? bv[j][ss] : b_base[(s0 + ss) * LDB + j * 32];
#pragma unroll
            for (int i = 0; i < WM; ++i) {
#pragma unroll
                for (int j = 0; j < WN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][ss], b[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    }
    __builtin_amdgcn_s_setprio(0);
}

// ---------------------------------------------------------------------------
// The same MFMAs with the chunk's last group of 4 k-steps carried over the
// barrier.  A group's operands (4 k-steps of WM A and WN B fragments) are
// read from LDS into a mt_mfma_group first; mt_mfma_tile_held reads group
// g + 1 while group g's MFMAs run, and leaves the last group's operands in
// `held`: the next chunk (or mt_mfma_group_run after the k loop) runs them
// first, after the barrier, so the matrix core has work while the waves
// leave the barrier and read the next chunk.  Per accumulator the products
// are added in the same k order as mt_mfma_tile, so the results are
// identical.  The barrier's release fence waits for the LDS reads into
// `held` (lgkmcnt(0)) before another wave may overwrite the buffer.
// ---------------------------------------------------------------------------

template <int WM, int WN>
struct mt_mfma_group {
    mt_f32x4 a[WM];
    mt_f32x4 b[WN];
};

template <int WM, int WN, int TK, int LDA, int LDB, bool ASWZ, bool BNM>
MT_INLINE void mt_mfma_group_load(const float* __restrict__ As, const float* __restrict__ Bs, unsigned lane,
                                  int s0, mt_mfma_group<WM, WN>& g) {
    constexpr int HALF = TK / 2;
    const unsigned li = lane & 31u;
    const unsigned lh = lane >> 5;
    unsigned m = 0u;
    if constexpr (ASWZ || BNM) m = mt_swz<TK / 4>(li);
    const float* a_base = ASWZ ? As + li * TK : As + li * LDA + lh * HALF;
    const float* b_base = BNM ? Bs + li * TK : Bs + (lh * HALF) * LDB + li;
    const unsigned slot = (lh * HALF + (unsigned)s0) / 4u;
#pragma unroll
    for (int i = 0; i < WM; ++i)
        g.a[i] = ASWZ ? mt_ld4(a_base + i * 32 * TK + 4u * (slot ^ m)) : mt_ld4(a_base + i * 32 * LDA + s0);
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        if constexpr (BNM) {
            g.b[j] = mt_ld4(b_base + j * 32 * TK + 4u * (slot ^ m));
        } else {
#pragma unroll
            for (int ss = 0; ss < 4; ++ss) g.b[j][ss] = b_base[(s0 + ss) * LDB + j * 32];
        }
    }
}

template <int WM, int WN>
MT_INLINE void mt_mfma_group_run(const mt_mfma_group<WM, WN>& g, mt_f32x16 (&acc)[WM][WN]) {
#pragma unroll
    for (int ss = 0; ss < 4; ++ss)
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(g.a[i][ss], g.b[j][ss], acc[i][j], 0, 0, 0);
}

// Runs `held` (the previous chunk's last group) first when has_held, then
// groups 0 .. G-2 of this chunk, and leaves group G-1's operands in `held`.
template <int WM, int WN, int TK, int LDA, int LDB, bool ASWZ = false, bool BNM = false>
MT_INLINE void mt_mfma_tile_held(const float* __restrict__ As, const float* __restrict__ Bs,
                                 mt_f32x16 (&acc)[WM][WN], unsigned lane, mt_mfma_group<WM, WN>& held,
                                 bool has_held) {
    constexpr int G = TK / 8;
    static_assert(TK % 8 == 0 && G >= 2, "a held group needs at least two groups of 4 k-steps per chunk");
    static_assert(LDA % 4 == 0, "LDA must keep 16-byte alignment");
    static_assert(!ASWZ || LDA == TK, "a swizzled A tile is dense");
    static_assert(!BNM || LDB == TK, "an n-major B tile is dense");
    __builtin_amdgcn_s_setprio(1);
    mt_mfma_group<WM, WN> f[G - 1];
    mt_mfma_group_load<WM, WN, TK, LDA, LDB, ASWZ, BNM>(As, Bs, lane, 0, f[0]);
    if (has_held) mt_mfma_group_run<WM, WN>(held, acc);
#pragma unroll
    for (int g = 0; g < G - 1; ++g) {
        if (g + 1 < G - 1)
            mt_mfma_group_load<WM, WN, TK, LDA, LDB, ASWZ, BNM>(As, Bs, lane, 4 * (g + 1), f[g + 1]);
        else
            mt_mfma_group_load<WM, WN, TK, LDA, LDB, ASWZ, BNM>(As, Bs, lane, 4 * (g + 1), held);
        mt_mfma_group_run<WM, WN>(f[g], acc);
    }
    __builtin_amdgcn_s_setprio(0);
}

// ---------------------------------------------------------------------------
// Row-owning waves for matmuls 128 columns wide.  Each of a workgroup's 16
// waves owns 16 rows x all 128 columns of a 256 x 128 tile, computed with
// v_mfma_f32_16x16x4f32 (D[16x16] += A[16x4] * B[4x16]; lane l supplies
// A[l%16][l/16] and B[l/16][l%16] and holds D[4 (l/16) + i][l%16], i < 4).
// A wave's A rows are its own: they go from global memory straight into the
// registers the MFMAs take (a prologue applied there), and only B is staged
// in LDS, as 64-wide k-chunks in two stages (64 KiB).
//   k: lane group g = l/16 takes a chunk's columns 16 g .. 16 g + 15, one per
//      step, so its A values are 16 consecutive floats (four 128-bit loads);
//   n: column block j < 4 puts lane column c = l%16 at output column 4 c + j,
//      block j >= 4 at 64 + 4 c + (j - 4), so a step's 8 B values are two
//      128-bit LDS reads (256 contiguous bytes per 16 lanes, no bank
//      conflicts) and each output row is stored 128 bits at a time.
// ---------------------------------------------------------------------------

struct mt_rw_group {
    mt_f32x4 b[2][2];  // [step][column half]
};

MT_INLINE void mt_rw_group_load(mt_rw_group& g, const float* __restrict__ Bs, unsigned krow0, unsigned c) {
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
        g.b[ss][0] = mt_ld4(Bs + (krow0 + (unsigned)ss) * 128u + 4u * c);
        g.b[ss][1] = mt_ld4(Bs + (krow0 + (unsigned)ss) * 128u + 64u + 4u * c);
    }
}

template <typename P>
MT_INLINE void mt_rw_group_run(const mt_rw_group& g, float a0, float a1, P pa, mt_f32x4 (&acc)[8]) {
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
        const float a = pa(ss == 0 ? a0 : a1);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, g.b[ss][0][j], acc[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[4 + j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, g.b[ss][1][j], acc[4 + j], 0, 0, 0);
    }
}

// One 64-wide chunk from the B stage at Bs (rows of 128 floats) and this
// lane's 16 A values `a` (raw; pa applies the prologue): 8 groups of 2
// steps, each group's B values read while the previous group's MFMAs run
// (the order pinned with sched_barrier: left alone, the compiler reads each
// value just before its MFMA and waits for it there).
template <typename P>
MT_INLINE void mt_rw_chunk(const mt_f32x4 (&a)[4], const float* __restrict__ Bs, P pa, unsigned lane,
                           mt_f32x4 (&acc)[8]) {
    const unsigned c = lane & 15u;
    const unsigned k0 = 16u * (lane >> 4);
    __builtin_amdgcn_s_setprio(1);
    mt_rw_group f[8];
    mt_rw_group_load(f[0], Bs, k0, c);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        if (g + 1 < 8) mt_rw_group_load(f[g + 1], Bs, k0 + 2u * (unsigned)(g + 1), c);
        __builtin_amdgcn_sched_barrier(0);
        mt_rw_group_run(f[g], a[g / 2][2 * (g % 2)], a[g / 2][2 * (g % 2) + 1], pa, acc);
        __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
}

// This lane's A values of the chunk at k0: arow points at its row's column
// 16 (lane / 16).
MT_INLINE void mt_rw_load(mt_f32x4 (&a)[4], const float* __restrict__ arow, unsigned k0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] = mt_ld4(arow + k0 + 4u * (unsigned)q);
}

// ---------------------------------------------------------------------------
// K-resident row waves for matmuls with a short K (64 or 128) whose B is read
// along K (n-major: B[k][n] at n * ldb + k, such as the transposed view K^T
// of attention scores).  Each of a workgroup's 16 waves owns 16 rows of a
// 256-row block and keeps those rows' whole K in registers (K/4 floats per
// lane, loaded once).  B streams through LDS in 128-column chunks, n-major
// [128][K], two stages; each chunk is a finished 256 x 128 output tile, 8
// column blocks of v_mfma_f32_16x16x4f32 per wave, stored with 128-bit
// stores issued between the MFMAs of the next column half.
//   k: lane group g = l/16 takes k = g K/4 + s at step s < K/4, so its A
//      values are K/4 consecutive floats of its row (128-bit loads), and its
//      B values of 4 consecutive steps are one 128-bit LDS read, logical
//      16-byte slot g K/16 + t (t = s/4) of the B row;
//   n: column block j puts lane column c = l%16 at output column
//      64 (j/4) + 4c + j%4, so blocks 4h .. 4h + 3 give a lane 4 consecutive
//      output columns of each of its rows (a 128-bit store; 256 contiguous
//      bytes per 16 lanes);
//   LDS: B row n (K/4 slots) holds logical slot L at physical slot
//      L ^ mt_kr_swz(n).  gfx950 serves a ds_read_b128 in 4 passes of 16
//      lanes, each pass two 8-lane groups k and k ^ 3 of one half-wave
//      (lanes 0-7 with 24-31, 8-15 with 16-23, ...), from 64 4-byte banks
//      (byte address mod 256) -- measured with rocprof's LDS bank-conflict
//      counter on fixed lane/address patterns.  Lane (g, c) reads row
//      64 (j/4) + 4c + j%4 at logical slot g K/16 + t, and a pass holds
//      lanes c < 8 of one g with lanes c >= 8 of g ^ 1.  So mt_kr_swz(n) is
//      c mod 8 for K = 128 (bit 3 of the slot then follows g) and c for
//      K = 64 (bit 3 follows c): the 16 lanes of every pass hit 16
//      distinct 16-byte bank groups.
// ---------------------------------------------------------------------------

template <int K>
MT_HD unsigned mt_kr_swz(unsigned n) {
    static_assert(K == 64 || K == 128, "K-resident rows hold K = 64 or 128");
    return (n >> 2) & (K == 128 ? 7u : 15u);
}

// Where wave-load `inst`, lane `lane` of the B loader puts its 16 bytes: row r
// of the [128][K] chunk, physical slot p = (64 inst + lane) mod K/4; it loads
// the row's logical slot p ^ mt_kr_swz(r).
template <int K>
MT_HD void mt_kr_slot(unsigned inst, unsigned lane, unsigned& r, unsigned& logical) {
    constexpr unsigned S = K / 4;
    const unsigned slot = inst * 64u + lane;
    r = slot / S;
    logical = (slot % S) ^ mt_kr_swz<K>(r);
}

// 128 n-major B rows of K floats (row stride ldb floats, a multiple of 4)
// into a dense swizzled LDS chunk [128][K] by direct-to-LDS loads; each
// lane's byte offsets from the chunk origin are computed once.
template <int K, int NT>
struct mt_kr_dma {
    static constexpr int S = K / 4;
    static constexpr int INSTR = 128 * S / 64;
    static constexpr int PERW = INSTR / (NT / 64);
    static_assert(INSTR % (NT / 64) == 0, "the chunk must split into the same number of wave loads per wave");
    unsigned off[PERW];
    unsigned lds_off;

    MT_INLINE mt_kr_dma(unsigned ldb, unsigned tid) {
        const unsigned lane = tid & 63u;
        const unsigned wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        lds_off = wave * PERW * 1024u;
#pragma unroll
        for (int q = 0; q < PERW; ++q) {
            unsigned r, logical;
            mt_kr_slot<K>(wave * PERW + q, lane, r, logical);
            off[q] = (r * ldb + 4u * logical) * 4u;
        }
    }

    // B rows n0 .. n0 + 127 of src (B[k][n] = src[n * ldb + k]).
    MT_INLINE void fetch(const float* __restrict__ src, unsigned ldb, unsigned n0, float* lds) const {
        const unsigned long long origin = mt_uniform_addr(src + (size_t)n0 * ldb);
        const unsigned base = __builtin_amdgcn_readfirstlane(mt_lds_addr(lds)) + lds_off;
#pragma unroll
        for (int q = 0; q < PERW; ++q) mt_dma16(origin, off[q], base + (unsigned)q * 1024u);
    }
};

// The B values of one group: quad t (4 steps), column half h (blocks
// 4h .. 4h + 3): rows 64h + 4c + jj of the chunk, logical slot g K/16 + t.
struct mt_kr_group {
    mt_f32x4 b[4];
};

template <int K>
MT_INLINE mt_f32x4 mt_kr_b(const float* __restrict__ bl, unsigned phys_slot, int h, int jj) {
    return mt_ld4(bl + (unsigned)(64 * h + jj) * K + 4u * phys_slot);
}

struct mt_kr_no_hook {
    MT_INLINE void operator()(int) const {}
};

// One 128-column chunk from the B stage at Bs and this lane's K/4 A values
// (already transformed by any prologue), column half by column half: groups
// q = 0 .. K/8 - 1 are quad t = q mod K/16 of half h = q / (K/16), 16 MFMAs
// each, steps 0 .. 3 in turn over the half's 4 blocks.  The group's B
// values sit in one set of 16 registers: block jj's value for the next
// group is read right after its step-3 MFMA (the order pinned with
// sched_barrier; measured on C5 S, as fast as two register sets, which
// cost 15 more VGPRs).  hook(q) runs after
// group q's MFMAs are issued -- the kernel stores one row of the other
// half's finished accumulators there, so the stores go out between MFMAs.
// The k order per output element is fixed: quads t = 0 .. K/16 - 1, steps
// 0 .. 3 within each.
template <int K, typename H = mt_kr_no_hook>
MT_INLINE void mt_kr_chunk(const mt_f32x4 (&a)[K / 16], const float* __restrict__ Bs, unsigned lane,
                           mt_f32x4 (&acc)[8], H hook = H{}) {
    constexpr int T = K / 16;
    const unsigned c = lane & 15u;
    const unsigned g = lane >> 4;
    const float* __restrict__ bl = Bs + 4u * c * (unsigned)K;
    const unsigned sw = mt_kr_swz<K>(4u * c);  // the same for every row this lane reads
    __builtin_amdgcn_s_setprio(1);
    mt_kr_group f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) f.b[jj] = mt_kr_b<K>(bl, (g * (unsigned)T) ^ sw, 0, jj);
#pragma unroll
    for (int q = 0; q < 2 * T; ++q) {
        const int h = q / T, t = q % T;
        const int hn = (q + 1) / T, tn = (q + 1) % T;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ss = 0; ss < 3; ++ss)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                acc[4 * h + jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][ss], f.b[jj][ss], acc[4 * h + jj], 0, 0, 0);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            acc[4 * h + jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][3], f.b[jj][3], acc[4 * h + jj], 0, 0, 0);
            if (q + 1 < 2 * T) f.b[jj] = mt_kr_b<K>(bl, (g * (unsigned)T + (unsigned)tn) ^ sw, hn, jj);
        }
        __builtin_amdgcn_sched_barrier(0);
        hook(q);
    }
    __builtin_amdgcn_s_setprio(0);
}

// Raw buffer access to an output of `bytes` bytes: one descriptor per
// workgroup (32-bit data, stride 0), so a store takes one per-lane byte
// offset and one wave-uniform one instead of a 64-bit address per lane; the
// hardware drops a store beyond the range instead of writing it.
typedef unsigned mt_u32x4 __attribute__((ext_vector_type(4)));

MT_INLINE mt_u32x4 mt_raw_buffer(const void* p, unsigned bytes) {
    const unsigned long long a = mt_uniform_addr(static_cast<const float*>(p));
    return mt_u32x4{(unsigned)a, (unsigned)(a >> 32) & 0xffffu, (unsigned)__builtin_amdgcn_readfirstlane((int)bytes), 0x00020000u};
}

// 16 bytes to rs + voff + soff (POLICY 16: sc1, device scope, written
// through the L2; 0: default).  The store reads its data registers after
// it issues, so nothing may write them in the next cycles: on MI355X a
// v_mul writing the first data register right after a 128-bit buffer store
// (the compiler inserts no wait state for a buffer store with an SGPR
// soffset) let the store write the new value in lanes 12-15 of a 16-lane
// group -- the next row's score in C5 S, in 16-32 elements per run.  The
// store is therefore issued here with two wait states behind it.
template <int POLICY = 0>
MT_INLINE void mt_buffer_store4(mt_f32x4 v, mt_u32x4 rs, unsigned voff, unsigned soff) {
    const unsigned so = __builtin_amdgcn_readfirstlane(soff);
    if constexpr (POLICY == 16)
        asm volatile("buffer_store_dwordx4 %0, %1, %2, %3 offen sc1\n\ts_nop 1"
                     :
                     : "v"(v), "v"(voff), "s"(rs), "s"(so)
                     : "memory");
    else
        asm volatile("buffer_store_dwordx4 %0, %1, %2, %3 offen\n\ts_nop 1"
                     :
                     : "v"(v), "v"(voff), "s"(rs), "s"(so)
                     : "memory");
}

// Row (within a 32x32 output block) of accumulator register v held by `lane`;
// the column is lane % 32.
MT_INLINE unsigned mt_acc_row(int v, unsigned lane) {
    return 8u * (unsigned)(v >> 2) + 4u * (lane >> 5) + (unsigned)(v & 3);
}

MT_INLINE void mt_zero(mt_f32x16& a) {
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = 0.f;
}

// ---------------------------------------------------------------------------
// Stream-K schedule for a persistent matmul: T output tiles of C k-chunks on
// P workgroups.  The first DP = floor(T / P) * P tiles are data-parallel
// (workgroup w takes tiles w, w + P, ...).  The k-chunks of the remaining
// T - DP tiles -- U = (T - DP) * C units, tile-major -- are cut into P
// contiguous ranges of U / P units; range j goes to workgroup P - 1 - j.
// A workgroup walks its range first (at most a partial tile, whole tiles,
// a partial tile), then its data-parallel tiles.
//
// A tile split between ranges is finished by the workgroup whose range
// holds its chunk 0 (the owner).  The others (contributors) hold later
// chunks at the start of their ranges: they store their partial
// accumulators to the workspace, then raise their flag.  Ranges after the
// owner's belong to lower workgroup indices, so an owner only ever waits for
// workgroups dispatched before it, which did that work first.  The owner
// adds the partials in range order, so results are reproducible.
//
// Workspace: MT_WS_HEAD words of flags (one per workgroup, 0 = empty; word
// MT_WS_HEAD - 1 is the error word), then one partial tile per workgroup.
// Flags start at 0 and every owner clears the flags it consumed, so the
// next launch starts clean.  A wait gives up after MT_SK_SPIN_LIMIT polls
// and sets the error word instead of hanging; the host checks it.
// ---------------------------------------------------------------------------

#define MT_WS_HEAD 1024u
#define MT_SK_SPIN_LIMIT (1u << 22)
// The schedule is plain integer arithmetic, callable from host code too (the
// CPU test suite checks its coverage and wait order).

struct mt_stream_k {
    unsigned chunks, P, w, j, dp, sk0, nsk, ndp;
    unsigned long long U, lo, hi;

    MT_HD void init(unsigned tiles, unsigned chunks_, unsigned P_, unsigned w_) {
        chunks = chunks_, P = P_, w = w_;
        dp = (tiles / P) * P;
        U = (unsigned long long)(tiles - dp) * chunks;
        j = P - 1u - w;
        lo = U * j / P;
        hi = U * (j + 1u) / P;
        sk0 = (unsigned)(lo / chunks);
        nsk = hi > lo ? (unsigned)((hi - 1u) / chunks) - sk0 + 1u : 0u;
        ndp = dp > w ? (dp - w + P - 1u) / P : 0u;
    }
    MT_HD unsigned items() const { return nsk + ndp; }
    // Item `it`: output tile t, chunks [kb, ke).
    MT_HD void item(unsigned it, unsigned& t, unsigned& kb, unsigned& ke) const {
        if (it < nsk) {
            const unsigned st = sk0 + it;
            const unsigned long long ts = (unsigned long long)st * chunks;
            kb = (unsigned)((lo > ts ? lo : ts) - ts);
            ke = (unsigned)((hi < ts + chunks ? hi : ts + chunks) - ts);
            t = dp + st;
        } else {
            t = w + (it - nsk) * P;
            kb = 0u;
            ke = chunks;
        }
    }
    // Start unit of range jj (jj <= P).
    MT_HD unsigned long long range_lo(unsigned jj) const { return U * jj / P; }
    // The owner of the split tile whose units end at tend: the first range
    // at offset >= c (c >= 1) after its own that is non-empty and starts
    // before tend, as an offset (its workgroup is w - offset); 0 when none
    // is left.  (Ranges are empty when there are fewer units than ranges.)
    MT_HD unsigned contributor(unsigned c, unsigned long long tend) const {
        for (; j + c < P; ++c) {
            const unsigned long long a = range_lo(j + c);
            if (a >= tend) return 0u;
            if (range_lo(j + c + 1u) > a) return c;
        }
        return 0u;
    }
};

// The partial slot's base pointer passes through an empty asm statement, so
// the slot addresses are computed where they are used (the rare hand-over
// branches) and not hoisted out of the tile loop, where they would hold
// registers across the mainloop.
MT_INLINE float* mt_ws_slot_base(float* p) {
    asm volatile("" : "+s"(p));
    return p;
}
MT_INLINE unsigned* mt_ws_flag(float* ws, unsigned w) { return reinterpret_cast<unsigned*>(ws) + w; }
MT_INLINE unsigned* mt_ws_error(float* ws) { return reinterpret_cast<unsigned*>(ws) + (MT_WS_HEAD - 1u); }
MT_INLINE float* mt_ws_part(float* ws, unsigned w, unsigned tile_floats) {
    return mt_ws_slot_base(ws + MT_WS_HEAD + (size_t)w * tile_floats);
}

// Contributor: each wave waits for its own partial stores to complete
// (s_waitcnt on every counter), the workgroup meets at the barrier, then
// lane 0 alone publishes them with one agent-scope release store of the
// flag.  An agent-scope release writes back the XCD's L2; doing it once per
// hand-over instead of once per wave kept the C4 X @ W1 kernel at 2.7 ms
// instead of 3.0 ms.
MT_INLINE void mt_sk_signal(unsigned* flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0u) __hip_atomic_store(flag, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// Owner: lane 0 polls the contributor's flag with relaxed loads (bounded),
// then one agent-scope acquire fence (it invalidates the CU's L1 and the
// XCD's L2 once, not once per poll or per wave) and clears the flag for the
// next launch; the barrier orders every lane's partial loads after it.
MT_INLINE void mt_sk_wait(unsigned* flag, unsigned* error) {
    if (threadIdx.x == 0u) {
        unsigned n = 0u;
        while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
            if (++n >= MT_SK_SPIN_LIMIT) {
                __hip_atomic_store(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Row reduction of a matmul's output in its epilogue (the matmul -> reduction
// epilogue extension): the kernel that writes Y = A @ B (+ a register
// epilogue) also writes r[row] = op over Y[row][:], op one of sum (OP 0),
// max (1), min (2), product (3) with the row-reduction kernels' combines.
//
// 1. A wave holds WM x WN blocks of 32x32 values in the MFMA layout (lane l:
//    column l % 32 of each block, 16 rows per block, mt_acc_row).  Per lane,
//    the WN blocks of each row are combined in block order: 16 WM values.
// 2. Across the 32 lanes of each half-wave, halving exchanges over lane bits
//    0, 1, 2, 3, 4: a lane keeps the half of its values its bit selects,
//    sends the other half to the lane that differs in that bit and combines
//    what it receives into what it keeps; once a lane holds one value, the
//    remaining steps combine both lanes' values.  Lane l then holds
//    MT_RR_KEEP(WM) values, value k for wave row mt_rr_row<WM>(l, k).  The
//    low bits go first: their exchanges are the most numerous and DPP quad
//    permutes serve them within the VALU op; bits 2-4 go through ds_swizzle.
// 3. The waves that share rows combine through LDS in wave order, one value
//    per row of the tile (generated code).
// 4. Each tile publishes its row values in the workspace (after the
//    MT_WS_HEAD flag words); the workgroup that publishes a row block's last
//    tile combines the block's tiles in column order and writes r.
// Every step has a fixed order, so results are reproducible; max and min
// give the same values as the row-reduction kernel, sum and product round
// differently (another summation order).
// ---------------------------------------------------------------------------

#define MT_RR_KEEP(WM) ((16 * (WM)) >= 32 ? (16 * (WM)) / 32 : 1)

template <int OP>
MT_INLINE float mt_rr_op(float a, float b) {
    if constexpr (OP == 0) return a + b;
    else if constexpr (OP == 1) return fmaxf(a, b);
    else if constexpr (OP == 2) return fminf(a, b);
    else return a * b;
}

// v from the lane whose index differs from this lane's in the bits of M
// (M < 32): DPP quad permutes for 1 and 2, ds_swizzle in its bitmask mode
// (and 0x1F, xor M within each 32 lanes) for 4, 8 and 16.
template <unsigned M>
MT_INLINE float mt_xor_lanes(float v) {
    const int x = __float_as_int(v);
    int y;
    if constexpr (M == 1u)
        y = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
    else if constexpr (M == 2u)
        y = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
    else
        y = __builtin_amdgcn_ds_swizzle(x, (int)((M << 10) | 0x1Fu));
    return __int_as_float(y);
}

// Wave-tile row of value k that `lane` keeps after mt_wave_row_reduce<WM>.
template <int WM>
MT_HD unsigned mt_rr_row(unsigned lane, int k) {
    unsigned idx = 0u, n = 16u * (unsigned)WM;
    for (int b = 0; b <= 4; ++b) {
        if (n > 1u) {
            n >>= 1;
            if ((lane >> b) & 1u) idx += n;
        }
    }
    idx += (unsigned)k;
    const unsigned i = idx >> 4, r = idx & 15u;
    return 32u * i + 8u * (r >> 2) + 4u * (lane >> 5) + (r & 3u);
}

// One exchange step over lane bit M with N values per lane (N == 1: combine).
template <unsigned M, int N, int OP>
MT_INLINE void mt_rr_step(float* w, unsigned lane) {
    if constexpr (N > 1) {
        constexpr int H = N / 2;
        const bool hi = (lane & M) != 0u;
#pragma unroll
        for (int k = 0; k < H; ++k) {
            const float send = hi ? w[k] : w[k + H];
            const float keep = hi ? w[k + H] : w[k];
            w[k] = mt_rr_op<OP>(keep, mt_xor_lanes<M>(send));
        }
    } else {
        w[0] = mt_rr_op<OP>(w[0], mt_xor_lanes<M>(w[0]));
    }
}

template <int WM, int WN, int OP>
MT_INLINE void mt_wave_row_reduce(const mt_f32x16 (&val)[WM][WN], unsigned lane, float (&out)[MT_RR_KEEP(WM)]) {
    constexpr int V = 16 * WM;
    float w[V];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float x = val[i][0][r];
#pragma unroll
            for (int j = 1; j < WN; ++j) x = mt_rr_op<OP>(x, val[i][j][r]);
            w[16 * i + r] = x;
        }
    constexpr int N1 = V > 1 ? V / 2 : 1, N2 = N1 > 1 ? N1 / 2 : 1, N3 = N2 > 1 ? N2 / 2 : 1, N4 = N3 > 1 ? N3 / 2 : 1;
    mt_rr_step<1u, V, OP>(w, lane);
    mt_rr_step<2u, N1, OP>(w, lane);
    mt_rr_step<4u, N2, OP>(w, lane);
    mt_rr_step<8u, N3, OP>(w, lane);
    mt_rr_step<16u, N4, OP>(w, lane);
#pragma unroll
    for (int k = 0; k < MT_RR_KEEP(WM); ++k) out[k] = w[k];
}

// Publish this workgroup's tile values of a row block: every wave's stores
// complete, the workgroup meets, then lane 0 increments the block's counter
// with one agent-scope acquire-release add (the release writes back the
// XCD's L2; the acquire invalidates the caches before the combining loads).
// Returns true in every lane of the workgroup that published the block's
// last tile, which resets the counter to 0 for the next launch.
MT_INLINE bool mt_rr_publish(unsigned* counter, unsigned tiles, unsigned* flag_lds) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0u) {
        const unsigned old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old + 1u == tiles;
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag_lds = last ? 1u : 0u;
    }
    __syncthreads();
    return *flag_lds != 0u;
}

// Publish row block `blk`'s tile values written by this workgroup (a tile
// earlier: its stores completed long ago, so the publish's wait is short)
// and, in the workgroup that completes the block, combine the block's `tn`
// column tiles in order into out[m0 + t] for the rows below M.
template <int OP, unsigned TM, unsigned NT>
MT_INLINE void mt_rr_finish(float* ws, unsigned blk, unsigned tn, unsigned m0, unsigned M, float* out,
                            unsigned* flag_lds) {
    const float* part = ws + MT_WS_HEAD + (size_t)blk * tn * TM;
    if (mt_rr_publish(reinterpret_cast<unsigned*>(ws) + blk, tn, flag_lds)) {
        for (unsigned t = threadIdx.x; t < TM; t += NT) {
            if (m0 + t >= M) continue;
            float r = part[t];
            for (unsigned n = 1u; n < tn; ++n) r = mt_rr_op<OP>(r, part[(size_t)n * TM + t]);
            out[m0 + t] = r;
        }
    }
}
