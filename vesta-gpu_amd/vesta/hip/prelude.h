// Vesta device library for gfx950 (CDNA4, wave64). Prepended to every
// generated kernel; compiled at run time by hipRTC.
//
// fp16 <-> fp32 conversion, 128-bit weight loads, wave64 reductions, block
// reductions through LDS, the agent-scope grid barrier and the last-arriver
// counter used by split reductions. Stores are vector stores and atomics are
// vector-memory atomics; nothing here writes through the scalar cache.

#define VWAVE 64
#ifndef VBLOCK
#define VBLOCK 512
#endif
#define VNWAVE (VBLOCK / VWAVE)
#ifndef INFINITY
#define INFINITY __builtin_huge_valf()
#endif

typedef unsigned short vh_half;
typedef unsigned int vh_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int vh_u32x2 __attribute__((ext_vector_type(2)));
typedef float vh_f32x4 __attribute__((ext_vector_type(4)));
typedef float vh_f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h2f(vh_half h) { return (float)__builtin_bit_cast(_Float16, h); }
// Round to nearest even, as numpy's astype(float16).
__device__ __forceinline__ vh_half f2h(float f) { return __builtin_bit_cast(vh_half, (_Float16)f); }

// The low and high fp16 of a 32-bit word as fp32.
__device__ __forceinline__ float h2f_lo(unsigned w) { return h2f((vh_half)(w & 0xffffu)); }
__device__ __forceinline__ float h2f_hi(unsigned w) { return h2f((vh_half)(w >> 16)); }

// 16-byte loads (global_load_dwordx4). `nt` marks data read once per step
// (weights, cache rows): streamed with the nontemporal hint.
__device__ __forceinline__ vh_u32x4 ld16(const void* p) { return *(const vh_u32x4*)p; }
__device__ __forceinline__ vh_u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load((const vh_u32x4*)p);
}
__device__ __forceinline__ vh_u32x2 ld8(const void* p) { return *(const vh_u32x2*)p; }
__device__ __forceinline__ vh_u32x2 ld8_nt(const void* p) {
  return __builtin_nontemporal_load((const vh_u32x2*)p);
}

// Unpack 8 fp16 (one 16-byte word) into fp32.
__device__ __forceinline__ void unpack8(vh_u32x4 q, float* w) {
  w[0] = h2f_lo(q.x); w[1] = h2f_hi(q.x); w[2] = h2f_lo(q.y); w[3] = h2f_hi(q.y);
  w[4] = h2f_lo(q.z); w[5] = h2f_hi(q.z); w[6] = h2f_lo(q.w); w[7] = h2f_hi(q.w);
}
__device__ __forceinline__ void unpack4(vh_u32x2 q, float* w) {
  w[0] = h2f_lo(q.x); w[1] = h2f_hi(q.x); w[2] = h2f_lo(q.y); w[3] = h2f_hi(q.y);
}

// ---------------------------------------------------------------- reductions
__device__ __forceinline__ float op_sum(float a, float b) { return a + b; }
__device__ __forceinline__ float op_max(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ float op_min(float a, float b) { return fminf(a, b); }

// Lane exchanges. Partners within a row of 16 lanes move through DPP (a
// lane-permute of the source operand, no memory); across rows through
// ds_bpermute. DPP controls: quad_perm [1,0,3,2] swaps lanes 2k, 2k+1
// (partner i^1), quad_perm [2,3,0,1] partner i^2, row_ror:8 partner i^8
// within the row; row_half_mirror (i <-> 7-i) and row_mirror (i <-> 15-i)
// are used once every lane of a quad / half-row already holds the same value.
#define VH_DPP_XOR1 0xB1
#define VH_DPP_XOR2 0x4E
#define VH_DPP_ROR8 0x128
#define VH_DPP_HALF_MIRROR 0x141
#define VH_DPP_MIRROR 0x140
template <int CTRL>
__device__ __forceinline__ float vh_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Lanes i and i^16 (rows 0<->1, 2<->3), or i and i^32 (halves), both values in
// every lane, through v_permlane16_swap / v_permlane32_swap (no LDS): swapping
// v with itself gives rows (r0, r0, r2, r2) and (r1, r1, r3, r3), or halves
// (h0, h0) and (h1, h1).
#define VH_PAIR(NAME, SWAP)                                                            \
  template <typename F>                                                               \
  __device__ __forceinline__ float NAME(float v, F op) {                              \
    const unsigned u = __builtin_bit_cast(unsigned, v);                               \
    const auto p = SWAP(u, u, false, false);                                          \
    return op(__builtin_bit_cast(float, (unsigned)p[0]), __builtin_bit_cast(float, (unsigned)p[1])); \
  }
VH_PAIR(vh_pair16, __builtin_amdgcn_permlane16_swap)
VH_PAIR(vh_pair32, __builtin_amdgcn_permlane32_swap)

// Whole-wave combine without LDS: rows of 16 lanes as above, then row_bcast:15
// adds lane 15 of rows 0 and 2 into rows 1 and 3, row_bcast:31 lane 31 into
// rows 2 and 3, so lane 63 holds the wave's value; every lane gets it from there.
#define VH_DPP_BCAST15 0x142
#define VH_DPP_BCAST31 0x143
template <int CTRL, int ROWS>
__device__ __forceinline__ float vh_dpp_rows(float v, float ident) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, ident), __builtin_bit_cast(int, v),
                                                               CTRL, ROWS, 0xF, false));
}
#define VH_WAVE_ALL(NAME, OP, IDENT)                                       \
  __device__ __forceinline__ float NAME(float v) {                         \
    v = OP(v, vh_dpp<VH_DPP_XOR1>(v));                                     \
    v = OP(v, vh_dpp<VH_DPP_XOR2>(v));                                     \
    v = OP(v, vh_dpp<VH_DPP_HALF_MIRROR>(v));                              \
    v = OP(v, vh_dpp<VH_DPP_MIRROR>(v));                                   \
    v = OP(v, vh_dpp_rows<VH_DPP_BCAST15, 0xA>(v, IDENT));                 \
    v = OP(v, vh_dpp_rows<VH_DPP_BCAST31, 0xC>(v, IDENT));                 \
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63)); \
  }
VH_WAVE_ALL(wave_red_sum, op_sum, 0.0f)
VH_WAVE_ALL(wave_red_max, op_max, -INFINITY)
VH_WAVE_ALL(wave_red_min, op_min, INFINITY)

// Combine over groups of `width` consecutive lanes (width a power of two
// <= 64): afterwards every lane of a group holds the group's value.
#define VH_GROUP_RED(NAME, OP, ALL)                                        \
  __device__ __forceinline__ float NAME(float v, int width) {              \
    if (width >= 64) return ALL(v);                                        \
    if (width >= 2) v = OP(v, vh_dpp<VH_DPP_XOR1>(v));                     \
    if (width >= 4) v = OP(v, vh_dpp<VH_DPP_XOR2>(v));                     \
    if (width >= 8) v = OP(v, vh_dpp<VH_DPP_HALF_MIRROR>(v));              \
    if (width >= 16) v = OP(v, vh_dpp<VH_DPP_MIRROR>(v));                  \
    if (width >= 32) v = vh_pair16(v, OP);                                 \
    return v;                                                              \
  }
VH_GROUP_RED(group_red_sum, op_sum, wave_red_sum)
VH_GROUP_RED(group_red_max, op_max, wave_red_max)
VH_GROUP_RED(group_red_min, op_min, wave_red_min)

// Combine over lane bits [lo, 64) (lo a power of two): lanes that differ only
// in those bits end with the same value, each group of lo consecutive lanes
// keeping its own position.
#define VH_WAVE_RED(NAME, OP)                                              \
  __device__ __forceinline__ float NAME(float v, int lo) {                 \
    if (lo <= 1) v = OP(v, vh_dpp<VH_DPP_XOR1>(v));                        \
    if (lo <= 2) v = OP(v, vh_dpp<VH_DPP_XOR2>(v));                        \
    if (lo <= 4) v = OP(v, __shfl_xor(v, 4, 64));                          \
    if (lo <= 8) v = OP(v, vh_dpp<VH_DPP_ROR8>(v));                        \
    if (lo <= 16) v = vh_pair16(v, OP);                                    \
    if (lo <= 32) v = vh_pair32(v, OP);                                    \
    return v;                                                              \
  }
VH_WAVE_RED(wave_red_sum_hi, op_sum)
VH_WAVE_RED(wave_red_max_hi, op_max)
VH_WAVE_RED(wave_red_min_hi, op_min)



// Block barrier for LDS traffic only: waits for this wave's LDS operations,
// not for its global loads (loads issued ahead of time stay in flight).
__device__ __forceinline__ void vh_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Whole-block reduction; every thread gets the result. `red` is VNWAVE
// floats of LDS. Ends with the block synchronised.
#define VH_BLOCK_RED(NAME, WRED, OP)                                       \
  __device__ __forceinline__ float NAME(float v, float* red) {             \
    v = WRED(v);                                                           \
    vh_lds_sync();                                                         \
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;                \
    vh_lds_sync();                                                         \
    float r = red[0];                                                      \
    for (int w = 1; w < VNWAVE; ++w) r = OP(r, red[w]);                    \
    return r;                                                              \
  }
VH_BLOCK_RED(block_red_sum, wave_red_sum, op_sum)
VH_BLOCK_RED(block_red_max, wave_red_max, op_max)
VH_BLOCK_RED(block_red_min, wave_red_min, op_min)

// (value, index) pairs: the larger value wins, equal values go to the lower
// index. Every thread gets the block's pair; `rv`/`ri` are VNWAVE slots of LDS.
__device__ __forceinline__ void argmax_pair(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  for (int o = 32; o > 0; o >>= 1) argmax_pair(v, i, __shfl_xor(v, o, 64), __shfl_xor(i, o, 64));
}
__device__ __forceinline__ void block_argmax(float& v, int& i, float* rv, int* ri) {
  for (int o = 32; o > 0; o >>= 1) argmax_pair(v, i, __shfl_xor(v, o, 64), __shfl_xor(i, o, 64));
  vh_lds_sync();
  if ((threadIdx.x & 63) == 0) { rv[threadIdx.x >> 6] = v; ri[threadIdx.x >> 6] = i; }
  vh_lds_sync();
  v = rv[0]; i = ri[0];
  for (int w = 1; w < VNWAVE; ++w) argmax_pair(v, i, rv[w], ri[w]);
}

// ---------------------------------------------------------------- coherence
// Values one block writes and another reads within a launch never rely on
// cache maintenance: they are stored with agent-scope coherent stores (sc1,
// written through to the device-coherent level across XCDs) and read with
// agent-scope coherent loads (sc1). A writer waits for its stores to
// complete (drain) before it signals; a reader issues its loads after it has
// seen the signal. Barriers therefore need no L2 writeback or invalidate.
#define VH_SC1 16   // cache-policy bit of buffer loads/stores: agent-coherent

typedef __amdgpu_buffer_rsrc_t vh_rsrc;
// Raw buffer descriptor over `bytes` bytes at `base` (out-of-range reads give 0,
// out-of-range writes are dropped).
__device__ __forceinline__ vh_rsrc mk_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ float ldc(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ldc_i(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ldc_u(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc_i(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc_u(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// fp16 element `i` of a residue through its descriptor.
__device__ __forceinline__ float ldc_h(vh_rsrc r, unsigned i) {
  return h2f(__builtin_bit_cast(vh_half, __builtin_amdgcn_raw_buffer_load_b16(r, i * 2u, 0, VH_SC1)));
}
__device__ __forceinline__ void stc_h(vh_rsrc r, unsigned i, float v) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, f2h(v)), r, i * 2u, 0, VH_SC1);
}
// 16 / 8 bytes starting at fp16 element `i` (i a multiple of 8 / 4).
__device__ __forceinline__ vh_u32x4 ldc16_h(vh_rsrc r, unsigned i) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, i * 2u, 0, VH_SC1);
}
__device__ __forceinline__ vh_u32x2 ldc8_h(vh_rsrc r, unsigned i) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, i * 2u, 0, VH_SC1);
}

// Loads and stores through buffer descriptors: a 32-bit element offset per
// lane (one register per address) over a base held in scalar registers.
#define VH_NT 2     // cache-policy bit: nontemporal (streamed once)
__device__ __forceinline__ float ldcs(vh_rsrc r, unsigned i) {       // coherent fp32
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, i * 4u, 0, VH_SC1));
}
__device__ __forceinline__ void stcs(vh_rsrc r, unsigned i, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, i * 4u, 0, VH_SC1);
}
__device__ __forceinline__ float ldg_h(vh_rsrc r, unsigned i) {      // read-only residues
  return h2f(__builtin_bit_cast(vh_half, __builtin_amdgcn_raw_buffer_load_b16(r, i * 2u, 0, 0)));
}
__device__ __forceinline__ unsigned short ldg_raw16(vh_rsrc r, unsigned i) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, i * 2u, 0, 0);
}
__device__ __forceinline__ float ldg_f(vh_rsrc r, unsigned i) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, i * 4u, 0, 0));
}
__device__ __forceinline__ int ldg_i(vh_rsrc r, unsigned i) {
  return (int)__builtin_amdgcn_raw_buffer_load_b32(r, i * 4u, 0, 0);
}
// 16 / 8 / 4 bytes of fp16 starting at element i, streamed (nontemporal).
__device__ __forceinline__ vh_u32x4 ldg16_nt(vh_rsrc r, unsigned i) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, i * 2u, 0, VH_NT);
}
// The same 16 bytes with the default (temporal) policy: kept by the caches,
// for weights that are worth finding there at the next step.
__device__ __forceinline__ vh_u32x4 ldg16_t(vh_rsrc r, unsigned i) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, i * 2u, 0, 0);
}
__device__ __forceinline__ vh_u32x2 ldg8_nt(vh_rsrc r, unsigned i) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, i * 2u, 0, VH_NT);
}
__device__ __forceinline__ unsigned ldg4_nt(vh_rsrc r, unsigned i) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, i * 2u, 0, VH_NT);
}

// x / d from r = 1 / d (both correctly rounded): q = x * r is within an ulp
// of the quotient, and one residual step (exact through the fma) rounds it
// correctly (Markstein), so the result is the IEEE quotient for finite
// nonzero d and a quotient that neither overflows nor underflows.
__device__ __forceinline__ float vh_divr(float x, float d, float r) {
  const float q = x * r;
  return fmaf(fmaf(-q, d, x), r, q);
}

// Matrix cores: 16x16 fp32 tile += A (16 x 32 fp16) * B (32 x 16 fp16); lane l
// holds A[l % 16][8 (l / 16) ..+8], B[8 (l / 16) ..+8][l % 16] and the result
// rows 4 (l / 16) ..+4 of column l % 16.
typedef _Float16 vh_h8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ vh_f32x4 vh_mfma(vh_u32x4 a, vh_u32x4 b, vh_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(vh_h8, a), __builtin_bit_cast(vh_h8, b), c, 0, 0, 0);
}
// Eight floats as fp16 halves v = hi + lo: hi the nearest fp16, lo the nearest
// fp16 to the remainder v - hi (exact in fp32).
__device__ __forceinline__ void vh_split8(const float* v, vh_u32x4& hi, vh_u32x4& lo) {
  vh_h8 h, l;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    h[j] = (_Float16)v[j];
    l[j] = (_Float16)(v[j] - (float)h[j]);
  }
  hi = __builtin_bit_cast(vh_u32x4, h);
  lo = __builtin_bit_cast(vh_u32x4, l);
}

// The same with the remainder scaled by 2^11 before rounding (exact), so lo
// keeps 11 significant bits whatever the magnitude (an unscaled remainder of a
// value below ~0.03 is an fp16 subnormal): v = hi + lo / 2048 to 22 bits.
// Products with lo go to their own accumulator, scaled back at the end.
#define VH_LO_SCALE 2048.0f
__device__ __forceinline__ void vh_split8s(const float* v, vh_u32x4& hi, vh_u32x4& lo) {
  vh_h8 h, l;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    h[j] = (_Float16)v[j];
    l[j] = (_Float16)((v[j] - (float)h[j]) * VH_LO_SCALE);
  }
  hi = __builtin_bit_cast(vh_u32x4, h);
  lo = __builtin_bit_cast(vh_u32x4, l);
}

// The matrix-core path carries activations as fp16 halves, so a value beyond
// the largest fp16 (65504) cannot go in: the split would give an infinite hi
// half. True if any of the eight values is beyond it (or is not a number);
// callers then raise VH_ERR_RANGE in the error word, and the host (which
// reads the word after the launch) refuses the results.
#define VH_HALF_MAX 65504.0f
#define VH_ERR_RANGE 2u
__device__ __forceinline__ bool vh_beyond_half8(const float* v) {
  bool b = false;
#pragma unroll
  for (int j = 0; j < 8; ++j) b |= !(__builtin_fabsf(v[j]) <= VH_HALF_MAX);
  return b;
}

// hi + lo / 2048 for partial sums of the two halves (see vh_split8s).
__device__ __forceinline__ float vh_hilo(float h, float l) { return fmaf(l, 1.0f / VH_LO_SCALE, h); }

// Fixed-point accumulators: fp32 values summed exactly as 64-bit integers in
// units of 2^-32 (any order of atomic adds gives the same bits), read back as
// fp32. Element i of such a buffer is the 8 bytes at float index i of global
// scratch (i even).
#define VH_FX_SCALE 4294967296.0
__device__ __forceinline__ long long vh_f2fx(float v) { return (long long)rint((double)v * VH_FX_SCALE); }
__device__ __forceinline__ float vh_fx2f(long long q) { return (float)((double)q * (1.0 / VH_FX_SCALE)); }
__device__ __forceinline__ long long ldfx_raw(vh_rsrc r, unsigned i) {
  return __builtin_bit_cast(long long, __builtin_amdgcn_raw_buffer_load_b64(r, i * 4u, 0, VH_SC1));
}
__device__ __forceinline__ float fxld(vh_rsrc r, unsigned i) { return vh_fx2f(ldfx_raw(r, i)); }
__device__ __forceinline__ void fxst(vh_rsrc r, unsigned i, float v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(vh_u32x2, vh_f2fx(v)), r, i * 4u, 0, VH_SC1);
}
__device__ __forceinline__ void fxadd(float* S, unsigned i, float v) {
  __hip_atomic_fetch_add((unsigned long long*)(S + i), (unsigned long long)vh_f2fx(v), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
}
// n fixed-point values at float index off into LDS floats (16-byte loads).
__device__ __forceinline__ void stage_fx(float* dst, vh_rsrc S, unsigned off, int n) {
  const int nv = (n + 1) >> 1;
  for (int base = threadIdx.x; base < nv; base += VBLOCK * 8) {
    vh_u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      v[u] = base + u * VBLOCK < nv ? __builtin_amdgcn_raw_buffer_load_b128(S, (off + 4u * (unsigned)(base + u * VBLOCK)) * 4u, 0, VH_SC1)
                                    : vh_u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (base + u * VBLOCK < nv) {
        const int j = 2 * (base + u * VBLOCK);
        dst[j] = vh_fx2f(__builtin_bit_cast(long long, vh_u32x2{v[u].x, v[u].y}));
        if (j + 1 < n) dst[j + 1] = vh_fx2f(__builtin_bit_cast(long long, vh_u32x2{v[u].z, v[u].w}));
      }
  }
}

// A fixed-point sum kept in C copies, cs floats apart (adders spread over the
// copies; the value is the exact integer sum of the copies): element i, and n
// elements at float index off into LDS floats.
template <int C>
__device__ __forceinline__ float fxld_c(vh_rsrc r, unsigned i, unsigned cs) {
  long long a = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) a += ldfx_raw(r, i + (unsigned)c * cs);
  return vh_fx2f(a);
}
template <int C>
__device__ __forceinline__ void stage_fxc(float* dst, vh_rsrc S, unsigned off, int n, unsigned cs) {
  const int nv = (n + 1) >> 1;
  for (int base = threadIdx.x; base < nv; base += VBLOCK) {
    vh_u32x4 v[C];
#pragma unroll
    for (int c = 0; c < C; ++c)
      v[c] = __builtin_amdgcn_raw_buffer_load_b128(S, (off + (unsigned)c * cs + 4u * (unsigned)base) * 4u, 0, VH_SC1);
    long long a = 0, b = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      a += __builtin_bit_cast(long long, vh_u32x2{v[c].x, v[c].y});
      b += __builtin_bit_cast(long long, vh_u32x2{v[c].z, v[c].w});
    }
    dst[2 * base] = vh_fx2f(a);
    if (2 * base + 1 < n) dst[2 * base + 1] = vh_fx2f(b);
  }
}
// 16 zero bytes at float index i of a buffer (agent-coherent store).
__device__ __forceinline__ void stz4(vh_rsrc r, unsigned i) {
  __builtin_amdgcn_raw_buffer_store_b128(vh_u32x4{0u, 0u, 0u, 0u}, r, i * 4u, 0, VH_SC1);
}

// Wait until every memory operation this wave issued has completed. The
// signal fences keep the compiler from moving memory operations across it.
__device__ __forceinline__ void drain() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Block barrier after which global data written by any thread of the block
// is visible to every thread of the block.
__device__ __forceinline__ void block_sync() {
  drain();
  vh_lds_sync();
}

// Four floats of global scratch at float index i (a multiple of 4), coherent.
__device__ __forceinline__ vh_f32x4 ldc4(vh_rsrc r, unsigned i) {
  return __builtin_bit_cast(vh_f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, i * 4u, 0, VH_SC1));
}

// Copy n floats of global scratch starting at float index `off` (a multiple
// of 4) into LDS (16-byte aligned) with every thread of the block: 16-byte
// coherent loads, up to 8 in flight per thread; the tail past n reads zeros.
// Every block reads the same vector at about the same time: each block starts
// at its own rotation of it so the requests spread over memory channels.
__device__ __forceinline__ void stage_ldc4(float* dst, vh_rsrc S, unsigned off, int n) {
  const int nv = (n + 3) >> 2;
  const int rot = (int)((blockIdx.x * 37u) % (unsigned)nv);
  for (int base = threadIdx.x; base < nv; base += VBLOCK * 8) {
    vh_f32x4 v[8];
    int ix[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      int j = base + u * VBLOCK + rot;
      ix[u] = j >= nv ? j - nv : j;
      v[u] = base + u * VBLOCK < nv ? ldc4(S, off + 4u * (unsigned)ix[u]) : vh_f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (base + u * VBLOCK < nv) *(vh_f32x4*)(dst + 4 * ix[u]) = v[u];
  }
}

// Copy n floats of global scratch (coherent loads) into LDS with every
// thread of the block; each thread keeps 8 loads in flight.
__device__ __forceinline__ void stage_ldc(float* dst, const float* src, int n) {
  for (int base = threadIdx.x; base < n; base += VBLOCK * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = base + u * VBLOCK < n ? ldc(src + base + u * VBLOCK) : 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (base + u * VBLOCK < n) dst[base + u * VBLOCK] = v[u];
  }
}

// ---------------------------------------------------------------- grid sync
// Split-phase grid barrier over monotonic arrival counters, one per XCD
// (block b arrives on counter b % 8, one 128-byte line each; consecutive
// blocks are dispatched to consecutive XCDs). grid_arrive() publishes that
// everything the block stored so far is complete; grid_wait(k) returns once
// every block has arrived k times in this launch. Between the two a block may
// issue work that does not depend on other blocks (weight loads). Counters only
// grow during a launch; grid_exit() lets the last block out of the kernel zero
// them, so they are zero between launches.
#define VH_BAR_GROUPS 8
#define VH_BAR_LINE 32
#define VH_BAR_WORDS (VH_BAR_LINE * (VH_BAR_GROUPS + 2))
#define VH_SPIN_LIMIT (1u << 24)
__device__ __forceinline__ void grid_arrive(unsigned* bar) {
  drain();
  vh_lds_sync();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(bar + VH_BAR_LINE * (blockIdx.x % VH_BAR_GROUPS), 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
// Lanes 0..7 of the polling wave (the block's last wave, which never has
// loads issued ahead of time in flight, so its polls complete as soon as the
// counters answer) each watch one counter. A wait that does not end within
// VH_SPIN_LIMIT polls (seconds) gives up and raises the error word
// bar[VH_BAR_ERROR] (only a launch whose blocks are not all resident can get
// there); every other wait looks at that word once per VH_ERR_POLLS polls and
// stops waiting once it is set, so a broken launch ends soon. The host reads
// the word (Kernel.check) and discards the launch's results.
#define VH_POLL_WAVE (VNWAVE - 1)
#define VH_BAR_ERROR (VH_BAR_LINE * 9 + 1)
#define VH_ERR_POLLS 4096u

__device__ __forceinline__ void grid_wait(unsigned* bar, unsigned nblk, unsigned k) {
  if ((int)(threadIdx.x >> 6) == VH_POLL_WAVE) {
    const unsigned g = threadIdx.x & 63u;
    bool done = g >= VH_BAR_GROUPS || g >= nblk;
    const unsigned target = done ? 0u : k * ((nblk - g + VH_BAR_GROUPS - 1u) / VH_BAR_GROUPS);
    // one poll in flight per lane (each counter line is read by every block, so
    // more polls only queue at its memory channel); polls are atomic loads, so
    // the compiler neither merges nor hoists them
    const unsigned* cp = bar + VH_BAR_LINE * (done ? 0u : g);
    unsigned n = 0;
    while (true) {
      if (!done) done = ldc_u(cp) >= target;
      if (__all(done)) break;
      __builtin_amdgcn_s_sleep(1);
      if (++n > VH_SPIN_LIMIT) {
        if (g == 0) stc_u(bar + VH_BAR_ERROR, 1u);
        break;
      }
      if ((n % VH_ERR_POLLS) == 0u && __builtin_amdgcn_readfirstlane(ldc_u(bar + VH_BAR_ERROR)) != 0u) break;
    }
  }
  vh_lds_sync();
}
__device__ __forceinline__ void grid_sync(unsigned* bar, unsigned nblk, unsigned& k) {
  k += 1u;
  grid_arrive(bar);
  grid_wait(bar, nblk, k);
}
// Called by every block once it will wait no more: the last block to get
// here zeroes the arrival counters and the exit counter.
__device__ __forceinline__ void grid_exit(unsigned* bar, unsigned nblk) {
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned* ex = bar + VH_BAR_LINE * VH_BAR_GROUPS;
    if (__hip_atomic_fetch_add(ex, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nblk - 1u) {
      for (unsigned g = 0; g < VH_BAR_GROUPS; ++g) stc_u(bar + VH_BAR_LINE * g, 0u);
      stc_u(ex, 0u);
    }
  }
}

// Readiness flags, for a set of producer blocks feeding a set of consumer
// blocks without a grid barrier: block b publishes in flag line b (one
// 128-byte line each, from `flags`) how many producer points of this launch it
// has passed, once everything it stored before is complete; a consumer waits
// only for the producers it reads from. Flags only grow during a launch;
// grid_exit_flags() lets the last block out zero them.
__device__ __forceinline__ void flag_publish(unsigned* flags, unsigned k) {
  drain();
  vh_lds_sync();
  if (threadIdx.x == 0) stc_u(flags + VH_BAR_LINE * blockIdx.x, k);
}
// Until blocks a0 .. a0 + n0 - 1, a1 .. a1 + n1 - 1, .. (at most 4 ranges, at
// most 64 blocks in all; the bounds are the same for every thread of the
// block) have published k: lane g of the polling wave watches the g-th of
// them, with grid_wait's spin limit and error-word checks.
__device__ __forceinline__ void flag_wait(unsigned* bar, const unsigned* flags, unsigned k, int a0, int n0,
                                          int a1 = 0, int n1 = 0, int a2 = 0, int n2 = 0, int a3 = 0, int n3 = 0) {
  if ((int)(threadIdx.x >> 6) == VH_POLL_WAVE) {
    const int g = (int)(threadIdx.x & 63u);
    const int pid = g < n0 ? a0 + g
                  : g < n0 + n1 ? a1 + g - n0
                  : g < n0 + n1 + n2 ? a2 + g - n0 - n1
                  : g < n0 + n1 + n2 + n3 ? a3 + g - n0 - n1 - n2 : -1;
    bool done = pid < 0;
    const unsigned* cp = flags + VH_BAR_LINE * (done ? 0 : pid);
    unsigned n = 0;
    while (true) {
      if (!done) done = ldc_u(cp) >= k;
      if (__all(done)) break;
      __builtin_amdgcn_s_sleep(1);
      if (++n > VH_SPIN_LIMIT) {
        if (g == 0) stc_u(bar + VH_BAR_ERROR, 1u);
        break;
      }
      if ((n % VH_ERR_POLLS) == 0u && __builtin_amdgcn_readfirstlane(ldc_u(bar + VH_BAR_ERROR)) != 0u) break;
    }
  }
  vh_lds_sync();
}
// grid_exit() for a kernel with readiness flags: a block's flag stores are
// complete before it counts itself out, and the last block out zeroes the
// nblk flag lines too.
__device__ __forceinline__ void grid_exit_flags(unsigned* bar, unsigned nblk, unsigned* flags) {
  drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned* ex = bar + VH_BAR_LINE * VH_BAR_GROUPS;
    if (__hip_atomic_fetch_add(ex, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nblk - 1u) {
      for (unsigned g = 0; g < VH_BAR_GROUPS; ++g) stc_u(bar + VH_BAR_LINE * g, 0u);
      for (unsigned b = 0; b < nblk; ++b) stc_u(flags + VH_BAR_LINE * b, 0u);
      stc_u(ex, 0u);
    }
  }
}

// Split reductions: after storing its partial (coherent stores), a block
// arrives on counter *cnt; the block that brings it to `total` is the last
// and gets true; it then reads the other partials with coherent loads. The
// last arriver resets *cnt.
__device__ __forceinline__ bool last_arrival(unsigned* cnt, unsigned total, int* flag_sh) {
  drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int last = prev == total - 1u;
    if (last) stc_u(cnt, 0u);
    *flag_sh = last;
  }
  __syncthreads();
  return *flag_sh != 0;
}

__device__ __forceinline__ unsigned long long vh_clock() { return wall_clock64(); }

// The thread index as a value the compiler cannot see through: rebinding it
// at the top of a loop body keeps per-site address arithmetic inside the
// site instead of being hoisted out of the loop (which spills registers).
__device__ __forceinline__ int vh_opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}
