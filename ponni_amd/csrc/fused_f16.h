// FUSED path, fp16 / bf16 operands with fp32 accumulation.
//
// Register tile H<T,NT,E>::v[m][n] (4 elements of type E per lane) holds the
// same features as the fp32 tile -- lane l, element e <-> feature 16m + 4g + e,
// column col0 + 16n + c -- rounded to E.  A dense layer runs on
// v_mfma_f32_16x16x32_{f16,bf16}: step t contracts 32 features, lane group g,
// element j <-> feature phi(t, g, j) = 16(2t + j/4) + 4g + j%4, which is just
// the concatenation of the lane's own elements of tiles 2t and 2t+1, so the
// B operand needs no data movement.  The host packs A in the same order:
// 1 KB per (output tile, step), lane l holding W[phi(t, l/16, j)][16mo + l%16]
// for j = 0..7.  The fp32 accumulator of each output tile gets its epilogue
// (bias, activation) in fp32 and is rounded to E once, which is where the
// reference model materializes the state.
#pragma once

#include "fused_f32.h"

namespace ponni_hip {
namespace fused {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <class E> struct Vec;
template <> struct Vec<_Float16> {
  using x4 = f16x4;
  using x8 = f16x8;
  __device__ static floatx4 mfma(x8 a, x8 b, floatx4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <> struct Vec<__bf16> {
  using x4 = bf16x4;
  using x8 = bf16x8;
  __device__ static floatx4 mfma(x8 a, x8 b, floatx4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};

template <int T, int NT, class E>
struct H {
  typename Vec<E>::x4 v[T > 0 ? T : 1][NT];
};

template <class E>
__device__ inline typename Vec<E>::x4 round4(floatx4 v) {
  return __builtin_convertvector(v, typename Vec<E>::x4);
}

template <class E>
__device__ inline floatx4 widen4(typename Vec<E>::x4 v) {
  return __builtin_convertvector(v, floatx4);
}

// The lane's element pointer for row 4g, column col0 + c, opaque to the
// compiler so that every row is one 64-bit add of a uniform (SGPR) offset.
template <class E>
__device__ inline E* lane_ptr(E* p, int64_t ld, Lane const& L) {
  int64_t off = int64_t(4 * L.g) * ld + L.col0 + L.c;
  asm volatile("" : "+v"(off));
  return p + off;
}

// x [N, batch] (row stride ld) -> tile; rows >= N and columns >= batch read 0.
// Waves whose columns are all inside the batch (all but the last) load
// without per-element predication.
template <int N, int NT, class E>
__device__ inline H<(N + 15) / 16, NT, E> load_rows_h(E const* __restrict__ x, int64_t ld, Lane const& L) {
  constexpr int T = (N + 15) / 16;
  H<T, NT, E> s;
  E const* __restrict__ xl = lane_ptr(x, ld, L);
  if (L.col0 + 16 * NT <= L.batch) {
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int n = 0; n < NT; n++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          int const f = 16 * m + 4 * L.g + e;
          s.v[m][n][e] = (N % 16 == 0 || f < N) ? xl[int64_t(16 * m + e) * ld + 16 * n] : E(0.0f);
        }
    return s;
  }
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) {
      bool const col_ok = L.col0 + 16 * n + L.c < L.batch;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = 16 * m + 4 * L.g + e;
        s.v[m][n][e] = (f < N && col_ok) ? xl[int64_t(16 * m + e) * ld + 16 * n] : E(0.0f);
      }
    }
  return s;
}

// ---- input rows prefetched into LDS one tile ahead ----------------------
// A wave's input tile (rows 0..16T-1, columns col0 .. col0 + 16 NT - 1) is
// requested with global_load_lds_dwordx4: piece p = 64 i + l of instruction
// i fills row slot s = p / (2 NT), columns 8 (p % (2 NT)) .. +7, landing at
// buf + 8 p, so buf holds 16 NT columns per slot.  Within each block of 16
// slots, slot 4a + b holds row 4b + a (a 4 x 4 transpose): the tile's
// reader takes rows 4g + e in lane group g, which then sit in slots 4e + g,
// 16 NT elements apart instead of 4 x that, in four different LDS banks
// (row-major, all four groups read one bank).  Only whole tiles
// of a 16-byte aligned x with a row stride of a multiple of 8 elements are
// requested this way (the caller checks); rows >= N issue nothing.  The
// loads are asynchronous: the caller waits (vmcnt) before reading buf.
typedef __attribute__((address_space(3))) void* lds_ptr;

// One 16-byte global_load_lds_dwordx4 per lane: lane l's 16 bytes at g land
// in LDS at lds + 16 l (lds uniform across the wave, passed in M0).  Issued
// as inline asm so that the compiler's wait insertion does not see an LDS
// write it cannot place: it cannot tell apart regions of one LDS array
// addressed at run time (the staging slots), so after the builtin it waits
// for every outstanding request (vmcnt(0)) before the next read of the
// array -- the first fragment read of every chunk waited for the requests
// just made for two chunks ahead.  Every read of data requested here is
// ordered by the kernel's own explicit waits (a vmcnt that leaves only
// later requests outstanding, then a barrier where other waves' requests
// are read); the compiler's own vmcnt values stay correct, because vector
// memory loads complete in issue order and untracked requests only make
// them wait longer.  The s_nop is the wait state the hardware needs
// between the write of M0 and an LDS DMA, which the compiler inserts for
// its own instructions but not in front of inline asm.
__device__ inline void dma16(void const* g, void* lds) {
  unsigned const m0 = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<uint64_t>((lds_ptr)lds)));
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m0) : "memory");
}

template <int N, int NT, class E>
__device__ inline void prefetch_rows_lds16(E const* __restrict__ x, int64_t ld, Lane const& L,
                                           unsigned short* __restrict__ buf) {
  constexpr int T = (N + 15) / 16;
  constexpr int PR = 2 * NT;  // 16-byte pieces per row
  static_assert(16 * PR % 64 == 0, "whole instructions per tile");
#pragma unroll
  for (int i = 0; i < T * 16 * PR / 64; i++) {
    int const piece = 64 * i + L.lane;
    int const slot = piece / PR, k = piece % PR;
    int const r = (slot & ~15) | ((slot & 3) << 2) | ((slot >> 2) & 3);
    if (N % 16 == 0 || r < N)
      dma16(x + int64_t(r) * ld + L.col0 + 8 * k, buf + 64 * 8 * i);
  }
}

// The lane's tile elements from a prefetched buf (row f = 16m + 4g + e in
// slot 16m + 4e + g); rows >= N read 0.
template <int N, int NT, class E>
__device__ inline H<(N + 15) / 16, NT, E> load_rows_lds16(unsigned short const* __restrict__ buf, Lane const& L) {
  constexpr int T = (N + 15) / 16;
  H<T, NT, E> s;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = 16 * m + 4 * L.g + e;
        unsigned short const bits = buf[(16 * m + 4 * e + L.g) * (16 * NT) + 16 * n + L.c];
        s.v[m][n][e] = (N % 16 == 0 || f < N) ? __builtin_bit_cast(E, bits) : E(0.0f);
      }
  return s;
}

// Waits: every outstanding vector-memory operation of this wave (vmcnt(0)),
// or every outstanding LDS operation (lgkmcnt(0)).
__device__ inline void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }
__device__ inline void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

template <int N, int T, int NT, class E>
__device__ inline void store_rows_h(H<T, NT, E> const& s, E* __restrict__ y, int64_t ld, Lane const& L) {
  E* __restrict__ yl = lane_ptr(y, ld, L);
  bool const full = L.col0 + 16 * NT <= L.batch;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) {
      bool const col_ok = full || L.col0 + 16 * n + L.c < L.batch;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = 16 * m + 4 * L.g + e;
        if ((N % 16 == 0 || f < N) && col_ok) yl[int64_t(16 * m + e) * ld + 16 * n] = s.v[m][n][e];
      }
    }
}

// Transposed tile (a dense layer run with its MFMA operands swapped, fused
// dense_hs<..., TR = true>): lane l, element e <-> feature 16m + c, column
// col0 + 16n + 4g + e, so each lane's 4 elements are consecutive columns of
// one output row.  Whole tiles of an 8-byte aligned y with a row stride of a
// multiple of 4 elements (vec_ok) store them as one 8-byte write; otherwise
// element by element inside the batch.  Rows >= N are not written.
template <int N, int T, int NT, class E>
__device__ inline void store_rows_ht(H<T, NT, E> const& s, E* __restrict__ y, int64_t ld, Lane const& L,
                                     bool vec_ok) {
  bool const full = vec_ok && L.col0 + 16 * NT <= L.batch;
#pragma unroll
  for (int m = 0; m < T; m++) {
    int const f = 16 * m + L.c;
    if (N % 16 != 0 && f >= N) continue;
    E* __restrict__ yr = y + int64_t(f) * ld + L.col0 + 4 * L.g;
#pragma unroll
    for (int n = 0; n < NT; n++) {
      if (full) {
        *reinterpret_cast<typename Vec<E>::x4*>(yr + 16 * n) = s.v[m][n];
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (L.col0 + 16 * n + 4 * L.g + e < L.batch) yr[16 * n + e] = s.v[m][n][e];
      }
    }
  }
}

template <int T, int NT, class E>
__device__ inline S<T, NT> to_f32(H<T, NT, E> const& h) {
  S<T, NT> s;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] = widen4<E>(h.v[m][n]);
  return s;
}

template <class E, int T, int NT>
__device__ inline H<T, NT, E> to_h(S<T, NT> const& s) {
  H<T, NT, E> h;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) h.v[m][n] = round4<E>(s.v[m][n]);
  return h;
}


// ---- A fragments staged through LDS -------------------------------------
// The workgroup's waves share the A fragments of as many consecutive output
// tiles of a dense layer as fill a 32 KB slot (a "chunk"; 4 tiles of a
// 256-input layer, 16 of a 64-input one).  A plan's chunks, in the order
// its dense layers run them, form a cyclic table (chunk_tab: the chunk's
// parameter offset in floats and its fragment count); chunk k is computed
// from slot k % 3 while chunks k + 1 and k + 2 are in flight to the other
// two: at the start of chunk k every wave requests its share of chunk k + 2
// with global_load_lds_dwordx4 (16 B per lane straight into LDS, no
// registers), and at its end waits until only those requests are
// outstanding (vmcnt counts in issue order, so chunk k + 1, requested a
// chunk earlier, has landed), then a workgroup barrier.  Each fragment is
// read from L2 once per workgroup instead of once per wave, and a request
// has two chunks of work to arrive in.
constexpr int kSlotFrags = 32;  // 1 KB fragments per slot
constexpr int kSlots = 3;

template <class E>
struct Stage {
  typename Vec<E>::x8* __restrict__ slots;  // LDS: kSlots x kSlotFrags x 64 lanes
  E const* __restrict__ params;
  int const* __restrict__ tab;  // chunk c: tab[2c] float offset, tab[2c + 1] fragments
  int n;                        // chunks per tile
  int k;                        // chunk being computed
};

// Requests per wave and chunk: the same for every chunk (partial chunks
// repeat their last fragment), so a constant vmcnt covers exactly one chunk.
template <int WAVES>
constexpr int chunk_requests() {
  return (kSlotFrags + WAVES - 1) / WAVES;
}

template <int WAVES, class E>
__device__ inline void request_chunk(Stage<E> const& st, int kk, int wave, int lane) {
  static_assert(kSlotFrags % WAVES == 0, "every wave makes the same number of requests");
  int const c = kk % st.n;
  E const* __restrict__ src = st.params + 2 * st.tab[2 * c];
  int const nf = st.tab[2 * c + 1];
  int const slot = kk % kSlots;
#pragma unroll
  for (int r = 0; r < chunk_requests<WAVES>(); r++) {
    int const f = wave + WAVES * r;
    int const fs = f < nf ? f : nf - 1;  // (a repeat lands in an unused fragment of the slot)
    dma16(src + fs * 512 + lane * 8, st.slots + (slot * kSlotFrags + f) * 64);
  }
}

// vmcnt(n) with the other counters left alone (gfx9 s_waitcnt encoding).
template <int N>
__device__ inline void wait_vmem_n() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// Kernel prologue: chunks 0 and 1 requested, landed, visible.
template <int WAVES, class E>
__device__ inline void stage_begin(Stage<E>& st) {
  int const wave = wave_id(), lane = threadIdx.x & 63;
  st.k = 0;
  request_chunk<WAVES>(st, 0, wave, lane);
  request_chunk<WAVES>(st, 1, wave, lane);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
}

// dense_hs schedule (each measured against its alternatives on c4): output
// tiles computed kTileGroup at a time, each group's epilogue run after the
// next group's MFMAs, the MFMA phase at raised wave priority.
constexpr int kTileGroup = 2;
constexpr bool kDeferEpilogue = true;
constexpr bool kSetPrio = true;
// A fragments read PONNI_PIPE contraction steps ahead of their MFMAs, with
// a scheduling barrier after each step so that the compiler neither hoists
// the reads further (their registers) nor sinks them: what plans with one
// column tile per wave at two waves per SIMD use (320-512 features: 3-7 %
// faster).  0 (the default, two column tiles per wave): each step's
// fragments are read in the step, the compiler schedules freely.
#ifndef PONNI_PIPE
#define PONNI_PIPE 0
#endif
constexpr int kFragPipe = PONNI_PIPE;

struct NoHook {
  __device__ void operator()() const {}
};

// Dense layer on fp16/bf16 MFMA with LDS-staged A fragments; returns the
// 16-bit output state.  init(mo) seeds output tile mo's fp32 accumulator
// (zero, or a bias that then costs no VALU add); epi(mo, t, o) finishes tile
// mo: its remaining epilogue steps in fp32 on t, then the 16-bit result into
// o.  The layer's chunks are st.k, st.k + 1, ... (the chunk table lists them
// in this order).  TR runs the MFMAs with their operands swapped (the
// transposed product, same fragments): the output tile is then transposed
// (feature 16m + c, column 16n + 4g + e; store_rows_ht), which only a layer
// whose output goes straight to memory can use, seeded with SeedRowsT.
// hook() runs once, at the start of chunk HOOK_CH before the chunk's
// request, so the memory requests it makes have landed when that chunk
// ends.
template <int TI, int TO, int NT, int WAVES, bool TR = false, int HOOK_CH = -1, class E, class Init, class Epi,
          class Hook = NoHook>
__device__ inline H<TO, NT, E> dense_hs(H<TI, NT, E> const& in, Stage<E>& st, Lane const& L, Init init, Epi epi,
                                        Hook hook = Hook()) {
  using V8 = typename Vec<E>::x8;
  using V4 = typename Vec<E>::x4;
  constexpr int TS = (TI + 1) / 2;
  static_assert(TS <= kSlotFrags, "at most 1024 input features (one output tile per chunk)");
  constexpr int CT = kSlotFrags / TS;  // output tiles per chunk
  constexpr int NCH = (TO + CT - 1) / CT;
  // Tiles per group: GT must divide CT and TO (else one at a time); DEFER
  // runs a group's epilogue after the next group's MFMAs.
  constexpr int GT = (CT % kTileGroup == 0 && TO % kTileGroup == 0) ? kTileGroup : 1;
  constexpr bool DEFER = kDeferEpilogue;
  int const wave = wave_id();
  H<TO, NT, E> out;
  floatx4 prev[GT][NT];
#pragma unroll
  for (int ch = 0; ch < NCH; ch++) {
    int const t0 = ch * CT;
    if (ch == HOOK_CH) hook();
    request_chunk<WAVES>(st, st.k + 2, wave, L.lane);
    V8 const* __restrict__ sl = st.slots + (st.k % kSlots) * (kSlotFrags * 64) + L.lane;
    // GT output tiles at a time: GT * NT independent accumulation chains.
#pragma unroll
    for (int tt = 0; tt < CT; tt += GT) {
      int const mo0 = t0 + tt;
      if (mo0 < TO) {
        floatx4 acc[GT][NT];
#pragma unroll
        for (int q = 0; q < GT; q++) {
          floatx4 const seed = init(mo0 + q < TO ? mo0 + q : mo0);
#pragma unroll
          for (int n = 0; n < NT; n++) acc[q][n] = seed;
        }
        // The wave in its MFMA phase runs at raised priority, so the SIMD's
        // other wave fills the matrix pipe's shadow with its VALU epilogue
        // instead of both waves contending in the same phase.
        if (kSetPrio) __builtin_amdgcn_s_setprio(1);
        // Fragment ring: step t's fragments sit in a[t % (D + 1)].
        constexpr int D = kFragPipe;
        V8 a[D + 1][GT];
        auto read = [&](int t) {
#pragma unroll
          for (int q = 0; q < GT; q++)
            if (mo0 + q < TO) a[t % (D + 1)][q] = sl[((tt + q) * TS + t) * 64];
        };
#pragma unroll
        for (int t = 0; t < D && t < TS; t++) read(t);
#pragma unroll
        for (int t = 0; t < TS; t++) {
          if (t + D < TS) read(t + D);
          V8 const (&at)[GT] = a[t % (D + 1)];
#pragma unroll
          for (int n = 0; n < NT; n++) {
            V4 const lo = in.v[2 * t][n];
            V4 const hi = (2 * t + 1 < TI) ? in.v[(2 * t + 1 < TI) ? 2 * t + 1 : 2 * t][n]
                                           : V4{E(0.0f), E(0.0f), E(0.0f), E(0.0f)};
            V8 const b = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int q = 0; q < GT; q++)
              if (mo0 + q < TO) acc[q][n] = TR ? Vec<E>::mfma(b, at[q], acc[q][n]) : Vec<E>::mfma(at[q], b, acc[q][n]);
          }
          if (D > 0) __builtin_amdgcn_sched_barrier(0);
        }
        if (kSetPrio) __builtin_amdgcn_s_setprio(0);
        if (DEFER) {
          // The previous group's epilogue runs behind this group's MFMAs.
          if (mo0 > 0)
#pragma unroll
            for (int q = 0; q < GT; q++) epi(mo0 - GT + q, prev[q], out.v[mo0 - GT + q]);
#pragma unroll
          for (int q = 0; q < GT; q++)
#pragma unroll
            for (int n = 0; n < NT; n++) prev[q][n] = acc[q][n];
        } else {
#pragma unroll
          for (int q = 0; q < GT; q++)
            if (mo0 + q < TO) epi(mo0 + q, acc[q], out.v[mo0 + q]);
        }
      }
    }
    // Chunk k + 1 has landed in every wave once only this chunk's requests
    // are outstanding; the barrier also ends every wave's reads of slot k,
    // which chunk k + 3's requests (made after it) overwrite.
    wait_vmem_n<chunk_requests<WAVES>()>();
    __syncthreads();
    st.k++;
  }
  if (DEFER)
#pragma unroll
    for (int q = 0; q < GT; q++) epi(TO - GT + q, prev[q], out.v[TO - GT + q]);
  return out;
}

// Accumulator seeds for dense_hs: zero, or the per-feature vector b.
struct SeedZero {
  __device__ floatx4 operator()(int) const { return floatx4{0.0f, 0.0f, 0.0f, 0.0f}; }
};
struct SeedRows {
  float const* __restrict__ b;
  int g;
  __device__ floatx4 operator()(int mo) const { return ld4(b + 16 * mo + 4 * g); }
};
// Seeds of a transposed tile: feature 16 mo + c in every element.
struct SeedRowsT {
  float const* __restrict__ b;
  int c;
  __device__ floatx4 operator()(int mo) const {
    float const v = b[16 * mo + c];
    return floatx4{v, v, v, v};
  }
};

// Final rounding of an epilogue tile to the 16-bit state.
template <class E, int NT>
__device__ inline void tile_round(floatx4 const (&t)[NT], typename Vec<E>::x4 (&o)[NT]) {
#pragma unroll
  for (int n = 0; n < NT; n++) o[n] = round4<E>(t[n]);
}

// Stage `bytes` (a multiple of 16) from global memory into LDS, once per
// workgroup; the caller synchronizes before the first read.
__device__ inline void stage_bytes(void* __restrict__ lds, void const* __restrict__ src, int bytes) {
  floatx4* d = reinterpret_cast<floatx4*>(lds);
  floatx4 const* s4 = reinterpret_cast<floatx4 const*>(src);
  for (int i = threadIdx.x; i < bytes / 16; i += blockDim.x) d[i] = s4[i];
}

// Projection add: out = in + round(b + W^T saved) computed in fp32, rounded once.
// Rows >= N (padding) are set to zero: their zero weights times an infinite
// or NaN saved feature are NaN, which a later contraction would read.
template <int TK, int TO, int N, int NT, class E>
__device__ inline void proj_add_h(H<TO, NT, E>& cur, H<TK, NT, E> const& sv, E const* __restrict__ w,
                                  float const* __restrict__ bias, Lane const& L) {
  using V8 = typename Vec<E>::x8;
  using V4 = typename Vec<E>::x4;
  constexpr int TS = (TK + 1) / 2;
#pragma unroll
  for (int mo = 0; mo < TO; mo++) {
    floatx4 const bb = ld4(bias + 16 * mo + 4 * L.g);
    floatx4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) acc[n] = bb;
#pragma unroll
    for (int t = 0; t < TS; t++) {
      V8 const a = *reinterpret_cast<V8 const*>(w + (mo * TS + t) * 512 + L.lane * 8);
#pragma unroll
      for (int n = 0; n < NT; n++) {
        V4 const lo = sv.v[2 * t][n];
        V4 const hi = (2 * t + 1 < TK) ? sv.v[(2 * t + 1 < TK) ? 2 * t + 1 : 2 * t][n] : V4{E(0.0f), E(0.0f), E(0.0f), E(0.0f)};
        acc[n] = Vec<E>::mfma(a, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), acc[n]);
      }
    }
#pragma unroll
    for (int n = 0; n < NT; n++) {
      cur.v[mo][n] = round4<E>(widen4<E>(cur.v[mo][n]) + acc[n]);
      if constexpr (N % 16 != 0)
        if (mo == TO - 1)
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (16 * mo + 4 * L.g + e >= N) cur.v[mo][n][e] = E(0.0f);
    }
  }
}

template <int TA, int TB, int NT, class E>
__device__ inline H<TA + TB, NT, E> concat_h(H<TA, NT, E> const& a, H<TB, NT, E> const& b) {
  H<TA + TB, NT, E> s;
#pragma unroll
  for (int m = 0; m < TA; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] = a.v[m][n];
#pragma unroll
  for (int m = 0; m < TB; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[TA + m][n] = b.v[m][n];
  return s;
}

}  // namespace fused
}  // namespace ponni_hip
