// Vesta device library for gfx950 (CDNA4, wave64). Prepended to every
// generated kernel; compiled at run time by hipRTC.
//
// fp16 <-> fp32 conversion, 128-bit weight loads, wave64 reductions, block
// reductions through LDS, the agent-scope grid barrier and the last-arriver
// counter used by split reductions. Stores are vector stores and atomics are
// vector-memory atomics; nothing here writes through the scalar cache.

#define VWAVE 64
#define VBLOCK 256
#define VNWAVE 4
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

// Butterfly over lane bits [lo, 64): afterwards every lane of each group of
// lanes that differ only in those bits holds the group's combined value.
#define VH_WAVE_RED(NAME, OP)                                              \
  __device__ __forceinline__ float NAME(float v, int lo) {                 \
    for (int o = 32; o >= lo; o >>= 1) v = OP(v, __shfl_xor(v, o, 64));    \
    return v;                                                              \
  }
VH_WAVE_RED(wave_red_sum_hi, op_sum)
VH_WAVE_RED(wave_red_max_hi, op_max)
VH_WAVE_RED(wave_red_min_hi, op_min)

// Butterfly over lane bits [0, width): groups of `width` consecutive lanes.
#define VH_GROUP_RED(NAME, OP)                                             \
  __device__ __forceinline__ float NAME(float v, int width) {              \
    for (int o = width >> 1; o > 0; o >>= 1) v = OP(v, __shfl_xor(v, o, 64)); \
    return v;                                                              \
  }
VH_GROUP_RED(group_red_sum, op_sum)
VH_GROUP_RED(group_red_max, op_max)
VH_GROUP_RED(group_red_min, op_min)

__device__ __forceinline__ float wave_red_sum(float v) { return group_red_sum(v, 64); }
__device__ __forceinline__ float wave_red_max(float v) { return group_red_max(v, 64); }
__device__ __forceinline__ float wave_red_min(float v) { return group_red_min(v, 64); }

// Whole-block reduction; every thread gets the result. `red` is VNWAVE
// floats of LDS. Ends with the block synchronised.
#define VH_BLOCK_RED(NAME, WRED, OP)                                       \
  __device__ __forceinline__ float NAME(float v, float* red) {             \
    v = WRED(v);                                                           \
    __syncthreads();                                                       \
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;                \
    __syncthreads();                                                       \
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
__device__ __forceinline__ void block_argmax(float& v, int& i, float* rv, int* ri) {
  for (int o = 32; o > 0; o >>= 1) argmax_pair(v, i, __shfl_xor(v, o, 64), __shfl_xor(i, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) { rv[threadIdx.x >> 6] = v; ri[threadIdx.x >> 6] = i; }
  __syncthreads();
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
  __syncthreads();
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
// Two-level arrival: block b arrives on the counter of group b % 8 (one
// 128-byte line each); the last arriver of a group arrives on the top
// counter; the last of those publishes generation `gen` in bar[0], which
// every block's thread 0 polls. Counters are reset by their last arriver, so
// they are zero between launches. bar[0] keeps the last generation; the
// caller starts from the value it reads at kernel start and adds one per
// barrier (only thread 0's copy is used).
#define VH_BAR_GROUPS 8
#define VH_BAR_LINE 32
#define VH_BAR_WORDS (VH_BAR_LINE * (VH_BAR_GROUPS + 2))
__device__ __forceinline__ void grid_sync(unsigned* bar, unsigned nblk, unsigned& gen) {
  drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    gen += 1u;
    const unsigned ng = nblk < VH_BAR_GROUPS ? nblk : VH_BAR_GROUPS;
    const unsigned g = blockIdx.x % ng;
    const unsigned members = (nblk - g + ng - 1u) / ng;
    unsigned* gc = bar + VH_BAR_LINE * (2u + g);
    unsigned* top = bar + VH_BAR_LINE;
    if (__hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == members - 1u) {
      stc_u(gc, 0u);
      drain();
      if (__hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ng - 1u) {
        stc_u(top, 0u);
        drain();
        stc_u(bar, gen);
      }
    }
    while (ldc_u(bar) != gen) __builtin_amdgcn_s_sleep(1);
  }
  __syncthreads();
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
