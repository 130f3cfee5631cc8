// Shared device helpers for the gfx950 attention kernels: element types,
// the 32x32x16 MFMA wrappers, register layouts, RoPE on 8-element chunks and
// wave-level reductions.  gfx950 (CDNA4) only: wave64, 160 KiB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace af {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// Element types.  Data moves as raw 16-byte chunks (u32x4 = 8 elements); the
// traits convert chunks to/from fp32 and run the matching MFMA.
// ---------------------------------------------------------------------------
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

struct F16 {
  using T = _Float16;
  using V8 = f16x8;
  __device__ static inline float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  __device__ static inline float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  // one v_cvt_pk_f16_f32 (round to nearest even)
  __device__ static inline uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  }
  __device__ static inline uint16_t one(float a) {
    return __builtin_bit_cast(uint16_t, (_Float16)a);
  }
  __device__ static inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // lo += w.lo, hi += w.hi in fp32 (v_fma_mix_f32 reads the f16 halves)
  __device__ static inline void add_pair(uint32_t w, float& lo, float& hi) {
    asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]" : "+v"(lo) : "v"(w));
    asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(hi) : "v"(w));
  }
  // lo = w.lo, hi = w.hi in fp32 (starts two sums without zeroing them)
  __device__ static inline void first_pair(uint32_t w, float& lo, float& hi) {
    asm("v_fma_mix_f32 %0, %1, 1.0, 0 op_sel_hi:[1,0,0]" : "=v"(lo) : "v"(w));
    asm("v_fma_mix_f32 %0, %1, 1.0, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(hi) : "v"(w));
  }
  // acc += w.lo + w.hi in fp32: one v_dot2_f32_f16 against (1, 1).  The
  // products are exact and f16 denormals are kept, so the sum is the one two
  // v_fma_mix_f32 give, in one instruction; it co-issues with the MFMAs of
  // other waves like any other VALU instruction.
  __device__ static inline void dot_pair(uint32_t w, float& acc) {
    asm("v_dot2_f32_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(w), "s"(0x3c003c00u));
  }
  // acc = w.lo + w.hi
  __device__ static inline void dot_first(uint32_t w, float& acc) {
    asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(acc) : "v"(w), "s"(0x3c003c00u));
  }
  // Call after the last add_pair into four sums, before ordinary code reads
  // them.  The compiler's hazard recognizer keeps dependent asm statements
  // two wait states apart, but it does not look at a compiler-generated
  // reader of an asm result, which then could issue right behind the last
  // v_fma_mix_f32.  Tying the sums through the nop gives that reader the
  // same separation (a precaution; it costs two cycles per tile).
  __device__ static inline void sums_ready(float& a, float& b, float& c, float& d) {
    asm volatile("s_nop 1" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
  }
};

struct BF16 {
  using T = __bf16;
  using V8 = bf16x8;
  __device__ static inline float lo(uint32_t w) {
    return __builtin_bit_cast(float, w << 16);
  }
  __device__ static inline float hi(uint32_t w) {
    return __builtin_bit_cast(float, w & 0xffff0000u);
  }
  // one v_cvt_pk_bf16_f32 (round to nearest even)
  __device__ static inline uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  }
  __device__ static inline uint16_t one(float a) {
    return __builtin_bit_cast(uint16_t, (__bf16)a);
  }
  __device__ static inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
        0);
  }
  __device__ static inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
        0);
  }
  // lo += w.lo, hi += w.hi in fp32 (a bf16 is the top half of its fp32)
  __device__ static inline void add_pair(uint32_t w, float& lo, float& hi) {
    lo += __builtin_bit_cast(float, w << 16);
    hi += __builtin_bit_cast(float, w & 0xffff0000u);
  }
  // lo = w.lo, hi = w.hi in fp32
  __device__ static inline void first_pair(uint32_t w, float& lo, float& hi) {
    lo = __builtin_bit_cast(float, w << 16);
    hi = __builtin_bit_cast(float, w & 0xffff0000u);
  }
  // acc += w.lo + w.hi in fp32: one v_dot2_f32_bf16 against (1, 1)
  __device__ static inline void dot_pair(uint32_t w, float& acc) {
    asm("v_dot2_f32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(w), "s"(0x3f803f80u));
  }
  // acc = w.lo + w.hi
  __device__ static inline void dot_first(uint32_t w, float& acc) {
    asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(acc) : "v"(w), "s"(0x3f803f80u));
  }
  __device__ static inline void sums_ready(float& a, float& b, float& c, float& d) {
    asm volatile("s_nop 1" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
  }
};

// Unpack a 16-byte chunk into 8 floats / pack 8 floats into a chunk.
template <class E>
__device__ inline void unpack8(u32x4 c, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = E::lo(c[i]);
    f[2 * i + 1] = E::hi(c[i]);
  }
}
template <class E>
__device__ inline u32x4 pack8(const float* f) {
  u32x4 c;
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = E::pack(f[2 * i], f[2 * i + 1]);
  return c;
}

// ---------------------------------------------------------------------------
// 32x32x16 MFMA register layouts (wave64, lane l, half h = l / 32).
//   A operand (32 x 16): lane holds row l%32, k-slots 8h .. 8h+7.
//   B operand (16 x 32): lane holds column l%32, k-slots 8h .. 8h+7.
//   C/D (32 x 32, 16 fp32): register r holds row 8*(r/4) + 4h + (r%4),
//                            column l%32.
// A and B pair the same k-slot of the same lane half, so any consistent
// assignment of k indices to (h, slot) gives the same product.
//
// Score tiles are computed transposed, S^T = K * Q^T, with A-row i reading
// key row kperm(i) (bits 2 and 3 of i swapped).  Then accumulator register r
// of lane half h holds key 16*(r/8) + 8h + (r%8): the eight registers
// 8j..8j+7 of a half are eight consecutive keys, which is exactly the B
// operand of the P*V MFMA over keys 16j..16j+15 -- P^T feeds the second MFMA
// straight from registers.  The column (query) is l%32 in both.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int kperm(int i) {
  return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}
__device__ __forceinline__ int acc_key(int r, int h) {
  return 16 * (r >> 3) + 8 * h + (r & 7);
}
__device__ __forceinline__ int acc_row(int r, int h) {
  return 8 * (r >> 2) + 4 * h + (r & 3);
}

// Partner lane l ^ 32 (the other half of a 32-wide MFMA column).
__device__ __forceinline__ float xor32(float x) {
  return __shfl_xor(x, 32, 64);
}

// max(x[l], x[l ^ 32]) with one v_permlane32_swap (no LDS round trip): the
// swap of a register with itself returns {x[l], x[l^32]} in some order.
__device__ __forceinline__ float max_xor32(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}

// ---------------------------------------------------------------------------
// Buffer resources: raw (stride 0) buffers whose num_records bounds every
// load -- an offset at or past the end (or "negative", i.e. huge unsigned)
// returns zeros, so tile loads need neither clamps nor branches.
// ---------------------------------------------------------------------------
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, kBufferWord3);
}
__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}
// 16 bytes per lane from the buffer straight into LDS (buffer_load ... lds):
// lane l's bytes land at lds_base + 16 l.  lds_base must be wave-uniform.
// Kept out of templates: the host pass of a template that names this builtin
// rejects later instantiations of the same template.
__device__ __forceinline__ void buf_ld16_lds(__amdgpu_buffer_rsrc_t r, void* lds_base,
                                             uint32_t byte_off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base,
                                           16, byte_off, 0, 0, 0);
}

// 4 bytes per lane from the buffer straight into LDS: lane l's bytes land at
// lds_base + 4 l.
__device__ __forceinline__ void buf_ld4_lds(__amdgpu_buffer_rsrc_t r, void* lds_base, uint32_t byte_off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base,
                                           4, byte_off, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Transposed LDS read (ds_read_b64_tr_b16).  Within each 16-lane group,
// result lane L, element i is element (L % 4) of the 64-bit chunk addressed
// by source lane (L % 16) / 4 + 4 i.  Two reads therefore build the
// 32x32x16 A operand "row d, k-slots = 8 consecutive rows of a row-major
// tile" that an MFMA needs for V^T without a transposed copy in LDS; see
// tr_source_offset for the per-lane address.
// ---------------------------------------------------------------------------
typedef short s16x4 __attribute__((ext_vector_type(4)));

// The pointer is __restrict__ so the read carries alias-scope metadata: the
// compiler then does not hold it behind an s_waitcnt vmcnt(0) for every load
// into LDS still in flight (the kernels order those with explicit waits and
// barriers; without the qualifier each transposing read waited for the
// prefetch of the next tile).
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* __restrict__ p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// Element offset (within a row-major tile of pitch `pitch`) that source lane
// `lane` must address so that, after two ds_read_b64_tr_b16 (t = 0, 1), the
// wave holds the A operand X^T[32 db + l%32][keys 16 kk + 8 h + (0..7)] of a
// 32x32x16 MFMA, X being the (keys x dims) tile.
__device__ __forceinline__ int tr_source_offset(int lane, int t, int pitch) {
  const int row = 8 * (lane >> 5) + 4 * t + ((lane & 15) >> 2);
  const int col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  return row * pitch + col;
}

// ---------------------------------------------------------------------------
// RoPE, rotate-half convention (reference: attnfuse/rope_utils.py:57-73):
//   out[d]       = x[d] cos[d]       - x[d+D/2] sin[d]
//   out[d+D/2]   = x[d+D/2] cos[d+D/2] + x[d] sin[d+D/2]
// computed in fp32 and rounded once to the element type (the reference
// rounds the rotated tile to the input dtype before the dot product,
// attnfuse/compiler/codegen.py:126-135).
// ---------------------------------------------------------------------------
template <class E>
__device__ inline void rope_pair(u32x4& lo, u32x4& hi, u32x4 clo, u32x4 slo,
                                 u32x4 chi, u32x4 shi);

// fp16: written on half vectors so the compiler emits mixed-precision FMAs
// (f16 operands, exact products, each sum rounded to f32), then each result
// is rounded from f32 to f16.  The empty asm keeps the f32 rounding: without
// it the compiler may fold the final FMA and the conversion into one
// v_fma_mix{lo,hi}_f16, which rounds once, straight to f16, and then a key
// rotated here can differ in its last bit from the same row rotated by the
// forward's in-register query path (measured: it did, in a kernel that
// rotates several rows per thread).
template <>
__device__ inline void rope_pair<F16>(u32x4& lo, u32x4& hi, u32x4 clo, u32x4 slo,
                                      u32x4 chi, u32x4 shi) {
  const f16x8 xl = __builtin_bit_cast(f16x8, lo), xh = __builtin_bit_cast(f16x8, hi);
  const f16x8 cl = __builtin_bit_cast(f16x8, clo), sl = __builtin_bit_cast(f16x8, slo);
  const f16x8 ch = __builtin_bit_cast(f16x8, chi), sh = __builtin_bit_cast(f16x8, shi);
  f16x8 ol, oh;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = __builtin_fmaf((float)xh[i], -(float)sl[i], 0.f);
    const float b = __builtin_fmaf((float)xl[i], (float)sh[i], 0.f);
    float rl = __builtin_fmaf((float)xl[i], (float)cl[i], a);
    float rh = __builtin_fmaf((float)xh[i], (float)ch[i], b);
    asm("" : "+v"(rl), "+v"(rh));
    ol[i] = (_Float16)rl;
    oh[i] = (_Float16)rh;
  }
  lo = __builtin_bit_cast(u32x4, ol);
  hi = __builtin_bit_cast(u32x4, oh);
}

template <>
__device__ inline void rope_pair<BF16>(u32x4& lo, u32x4& hi, u32x4 clo, u32x4 slo,
                                       u32x4 chi, u32x4 shi) {
  float xl[8], xh[8], cl[8], sl[8], ch[8], sh[8], ol[8], oh[8];
  unpack8<BF16>(lo, xl);
  unpack8<BF16>(hi, xh);
  unpack8<BF16>(clo, cl);
  unpack8<BF16>(slo, sl);
  unpack8<BF16>(chi, ch);
  unpack8<BF16>(shi, sh);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    ol[i] = xl[i] * cl[i] - xh[i] * sl[i];
    oh[i] = xh[i] * ch[i] + xl[i] * sh[i];
  }
  lo = pack8<BF16>(ol);
  hi = pack8<BF16>(oh);
}

// Inverse (transpose) rotation applied to a gradient g of the rotated vector:
//   dx[d]     = g[d] cos[d] + g[d+D/2] sin[d+D/2]
//   dx[d+D/2] = g[d+D/2] cos[d+D/2] - g[d] sin[d]
__device__ inline void rope_grad_pair(float& glo, float& ghi, float clo,
                                      float slo, float chi, float shi) {
  float a = glo * clo + ghi * shi;
  float b = ghi * chi - glo * slo;
  glo = a;
  ghi = b;
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

// Byte range of `rows` rows of D elements at `rstride` elements apart.
template <int D>
__device__ __forceinline__ uint32_t span_bytes(int rows, int64_t rstride) {
  return rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * rstride + D) * 2) : 0u;
}

// ---------------------------------------------------------------------------
// LDS tile swizzle.  A tile row holds D elements = D/8 chunks of 16 bytes;
// logical chunk k of row r is stored at chunk k ^ lds_swz<D>(r).  The
// function depends on r mod 16 only, so tiles can be addressed at 16-row
// offsets without re-swizzling.  Chosen so that (a) 16 lanes reading the
// same chunk of 16 different rows (the MFMA row operands) and (b) the
// 32-lane passes of ds_read_b64_tr_b16 (4 rows x 4 consecutive chunks) each
// touch 64 distinct banks.
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ int lds_swz(int r) {
  if constexpr (D >= 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  else if constexpr (D == 64) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else return (r >> 2) & 3;
}
// element offset of element `col` of row `r`
template <int D>
__device__ __forceinline__ int lds_at(int r, int col) {
  return r * D + 8 * ((col >> 3) ^ lds_swz<D>(r)) + (col & 7);
}
// Per-lane offset of the two ds_read_b64_tr_b16 (t = 0, 1) that together
// give this lane the 32x32x16 A operand X^T[32 db + l%32][rows 8h .. 8h+7]
// of the first 16 rows of a row-major, swizzled (rows x D) tile -- the
// read pattern tr_source_offset describes for padded tiles.  Add 16*j*D
// for rows 16j .. 16j+15.
template <int D>
__device__ __forceinline__ int tr_at(int lane, int t, int db) {
  const int row = 8 * (lane >> 5) + 4 * t + ((lane & 15) >> 2);
  const int col = 32 * db + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  return lds_at<D>(row, col);
}

// Byte offset of element col of row `row` (16-bit elements, rows `stride`
// elements apart) in 32-bit arithmetic: buffer offsets stay below the 4 GiB
// range (checked on the host).  The empty asm keeps the multiply and the add
// apart: fused, they became a 64-bit multiply-add whose register pair the
// register allocator kept (and spilled) for the whole kernel.
__device__ __forceinline__ uint32_t dma_off(int row, int64_t stride, int col) {
  uint32_t prod = (uint32_t)row * (uint32_t)stride;
  asm("" : "+v"(prod));
  return (prod + (uint32_t)col) * 2u;
}

// Staging of two row tiles (rows [r0, r0 + ROWS) of tensors A and B, D
// elements each) straight from global memory into one swizzled LDS stage --
// tile A at element 0 of the stage, tile B at element ROWS * D -- with
// buffer_load ... lds: one wave instruction fills 64 consecutive 16-byte LDS
// chunks (lane l at chunk l), so each lane fetches the logical chunk that its
// slot holds under the swizzle.  No data passes through registers.  Rows past
// the end of a tensor fall outside its resource and load as zeros.
// off + delta computed next to the load that uses it: as plain C++ the
// compiler hoists the loop-invariant sums out of the stage loop and holds
// one register per load again.
__device__ __forceinline__ uint32_t add_at_use(uint32_t off, uint32_t delta) {
  uint32_t r;
  asm volatile("v_add_u32 %0, %1, %2" : "=v"(r) : "s"(delta), "v"(off));
  return r;
}

// A wave instruction covers RPI = 512 / D rows.  When a wave's instructions
// for one tensor lie a multiple of 16 rows apart (the swizzle repeats every
// 16 rows), their per-lane byte offsets differ by a wave-uniform row delta:
// the wave then keeps one offset register per tensor and adds the delta per
// load, instead of one register per instruction.  The delta stays in the
// vector offset, inside the hardware bounds check that zeroes rows past the
// end.
template <int D, int NT, int ROWS = 32>
struct TileDma {
  static_assert(ROWS % 16 == 0 && ROWS * D % 512 == 0, "whole wave instructions per tile");
  static constexpr int CHUNKS = ROWS * D / 8;        // per tensor, a multiple of 64
  static constexpr int INSTR = 2 * CHUNKS / 64;      // wave instructions per stage
  static constexpr int WAVES = NT / 64;
  static constexpr int IPW = (INSTR + WAVES - 1) / WAVES;
  static constexpr int RPI = 512 / D;
  // instructions i < IPW / 2 of every wave load tile A, the rest tile B
  static constexpr bool SHARED = (INSTR / 2) % WAVES == 0 && (RPI * WAVES) % 16 == 0;
  uint32_t off[SHARED ? 2 : IPW];                    // byte offsets within rows [r0, r0 + ROWS)

  __device__ static uint32_t lane_off(int m, int lane, int64_t astride, int64_t bstride) {
    const int pos = 64 * m + lane;
    const bool isb = pos >= CHUNKS;
    const int rem = isb ? pos - CHUNKS : pos;
    const int row = rem / (D / 8), kp = rem % (D / 8);
    return dma_off(row, isb ? bstride : astride, 8 * (kp ^ lds_swz<D>(row)));
  }
  __device__ void init(int w, int lane, int64_t astride, int64_t bstride) {
    if constexpr (SHARED) {
      off[0] = lane_off(w, lane, astride, bstride);
      off[1] = lane_off(w + INSTR / 2, lane, astride, bstride);
    } else {
#pragma unroll
      for (int i = 0; i < IPW; ++i) off[i] = lane_off(w + i * WAVES, lane, astride, bstride);
    }
  }
  // stage = element offset of the stage inside `lds`
  __device__ void load(uint16_t* lds, int stage, int w, const uint16_t* abase, int64_t astride, int an,
                       const uint16_t* bbase, int64_t bstride, int bn, int r0) const {
    const auto ar = make_rsrc(abase + (int64_t)r0 * astride, span_bytes<D>(an - r0, astride));
    const auto br = make_rsrc(bbase + (int64_t)r0 * bstride, span_bytes<D>(bn - r0, bstride));
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int m = w + i * WAVES;   // wave-uniform
      if (INSTR % WAVES != 0 && m >= INSTR) break;
      if constexpr (SHARED) {
        const bool isb = i >= IPW / 2;
        const int di = isb ? i - IPW / 2 : i;
        const uint32_t delta = (uint32_t)(di * RPI * WAVES * (isb ? bstride : astride) * 2);
        buf_ld16_lds(isb ? br : ar, lds + stage + 512 * m, di == 0 ? off[isb ? 1 : 0] : add_at_use(off[isb ? 1 : 0], delta));
      } else {
        buf_ld16_lds(64 * m >= CHUNKS ? br : ar, lds + stage + 512 * m, off[i]);
      }
    }
  }
};

// One tensor's rows [r0, r0 + ROWS) into a swizzled LDS tile, the same way.
template <int D, int NT, int ROWS>
struct RowsDma {
  static_assert(ROWS % 16 == 0 && ROWS * D % 512 == 0, "whole wave instructions per tile");
  static constexpr int CHUNKS = ROWS * D / 8;
  static constexpr int INSTR = CHUNKS / 64;
  static constexpr int WAVES = NT / 64;
  static constexpr int IPW = (INSTR + WAVES - 1) / WAVES;
  static constexpr int RPI = 512 / D;
  static constexpr bool SHARED = INSTR % WAVES == 0 && (RPI * WAVES) % 16 == 0;
  uint32_t off[SHARED ? 1 : IPW];

  __device__ static uint32_t lane_off(int m, int lane, int64_t stride) {
    const int pos = 64 * m + lane;
    const int row = pos / (D / 8), kp = pos % (D / 8);
    return dma_off(row, stride, 8 * (kp ^ lds_swz<D>(row)));
  }
  __device__ void init(int w, int lane, int64_t stride) {
    if constexpr (SHARED) {
      off[0] = lane_off(w, lane, stride);
    } else {
#pragma unroll
      for (int i = 0; i < IPW; ++i) off[i] = lane_off(w + i * WAVES, lane, stride);
    }
  }
  // tile = element offset of the tile inside `lds`
  __device__ void load(uint16_t* lds, int tile, int w, const uint16_t* base, int64_t stride, int n, int r0) const {
    const auto rs = make_rsrc(base + (int64_t)r0 * stride, span_bytes<D>(n - r0, stride));
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int m = w + i * WAVES;   // wave-uniform
      if (INSTR % WAVES != 0 && m >= INSTR) break;
      if constexpr (SHARED) {
        buf_ld16_lds(rs, lds + tile + 512 * m, i == 0 ? off[0] : add_at_use(off[0], (uint32_t)(i * RPI * WAVES * stride * 2)));
      } else {
        buf_ld16_lds(rs, lds + tile + 512 * m, off[i]);
      }
    }
  }
};

// Wait until this wave's loads into LDS have landed (the barrier after it
// then publishes the whole stage).
__device__ __forceinline__ void wait_lds_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Workgroup barrier over LDS tiles that leaves this wave's later loads into
// LDS in flight.  __syncthreads() is a release/acquire fence pair around
// s_barrier, and for the release the compiler waits for every outstanding
// vector memory operation (vmcnt(0)), the loads of stages still ahead
// included, which serialises any deeper prefetch.  Here the wave's own LDS
// accesses complete (lgkmcnt(0)) before s_barrier and the "memory" clobber
// keeps the compiler from moving memory accesses across it; loads into LDS
// that other waves read after the barrier are waited for (wait_vmcnt)
// before it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Wait until at most N vector memory operations of this wave are in flight
// (they complete in issue order): the loads of a later stage may stay
// outstanding while an earlier stage's have landed.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// ---------------------------------------------------------------------------
// Work item and (batch, head) of workgroup g of a grid of n_items x BH
// workgroups.  The dispatcher hands workgroup g to XCD g % 8, so with BH a
// multiple of 8 the default order (item-major, head-minor) keeps every head
// on one XCD, but an XCD then walks all BH / 8 of its heads at once.  With
// gh > 0 (BH a multiple of 8 gh) it walks them gh at a time, every item of
// a group before the next group, so that the rows a group's workgroups
// re-read (block-sparse walks load each listed tile once per list that
// names it) stay in the XCD's L2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void xcd_head_groups(int g, int BH, int n_items, int gh, int& item, int& bh) {
  if (gh <= 0) {
    bh = g % BH;
    item = g / BH;
    return;
  }
  const int x = g & 7, k = g >> 3, per = gh * n_items;
  const int grp = k / per, r = k - grp * per;
  item = r / gh;
  bh = x + 8 * (grp * gh + (r - item * gh));
}

// ---------------------------------------------------------------------------
// Entry e (wave-uniform) of one BlockMask row: list a, then list b.  The
// lists are read through the constant address space, so the compiler loads
// them with scalar loads (s_load_dword, counted by lgkmcnt).  Through a
// generic pointer it used a vector load, and the s_waitcnt vmcnt that
// consumed it also waited for every tile load into LDS still in flight: each
// step of a block-sparse loop stalled until the previous tiles had landed.
// ---------------------------------------------------------------------------
typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
__device__ inline int bs_row_get(const int32_t* a, int na, const int32_t* b, int e) {
  return e < na ? ((const_i32_ptr)a)[e] : ((const_i32_ptr)b)[e - na];
}

// The tile starts of one block-sparse walk, held in a register: lane l
// holds the start of tile l, read by a wave-uniform tile index with
// v_readlane.  Looked up per stage from the lists instead, every stage's K/V
// (or Q/dO) loads waited out a scalar load round trip and a division by the
// tiles per block first.  Tile t of the walk is sub-tile t % sub of entry
// e0 + t / sub (entries of `blk` rows or keys, sub-tiles of `tile`); tiles
// from 64 on (walks longer than a work plan's pieces) are looked up in the
// lists.  Bit 0 of a start (tile starts are multiples of 32) marks a tile of
// a partial block whose element mask applies.
struct BsTiles {
  int lo;             // lane l: start of tile l, + 1 if it is a masked partial tile
  const int32_t* a;
  const int32_t* b;
  const int32_t* flags;
  int na, e0, sub, blk, tile;
  int pmode;          // 0: no element masks; 1: entries >= na (list b) are
                      // partial; 2: entries e with flags[e] != 0 are

  __device__ bool part_of(int e) const {
    if (pmode == 1) return e >= na;
    if (pmode == 2) return ((const_i32_ptr)flags)[e] != 0;
    return false;
  }
  __device__ int raw_lookup(int t) const {
    const int e = t / sub;
    return bs_row_get(a, na, b, e0 + e) * blk + (t - e * sub) * tile + (part_of(e0 + e) ? 1 : 0);
  }
  // Lanes past the walk's last tile hold 0.  A lane's entry of list a (and
  // its partial flag) is loaded before the list count is known, inside the
  // padded row of `wa` entries: the count, read from memory in parallel,
  // then only selects.  Loaded after it instead, the entries added one
  // memory round trip to the start of every block-sparse workgroup (2500
  // cycles of the measured 6000 before a forward workgroup's first tile).
  // List b, which entries at or past the count come from, is read only by
  // the lanes that need it.
  __device__ void init(const int32_t* a_, int na_, const int32_t* b_, int e0_, int sub_, int blk_, int tile_,
                       int ntiles, int lane, int64_t wa, int pmode_ = 0, const int32_t* flags_ = nullptr) {
    a = a_;
    na = na_;
    b = b_;
    e0 = e0_;
    sub = sub_;
    blk = blk_;
    tile = tile_;
    pmode = pmode_;
    flags = flags_;
    const int e = e0 + lane / sub;
    // The entry index clamped into the row (wa >= 1, checked on the host):
    // every lane loads unconditionally.  A condition around the load made the
    // compiler emit an invalid aperture check in some instantiations.
    const int ec = (int)min<int64_t>(e, wa - 1);
    const int va = a[ec];
    const int fl = pmode == 2 ? flags[ec] : 0;
    if (lane >= ntiles) {
      lo = 0;
    } else {
      const bool part = pmode == 1 ? e >= na : fl != 0;
      lo = (e < na ? va : b[e - na]) * blk + (lane % sub) * tile + (part ? 1 : 0);
    }
  }
  __device__ __forceinline__ int raw(int t) const {
    if (t < 64) return __builtin_amdgcn_readlane(lo, t);
    return raw_lookup(t);
  }
  // first row (key or query) of tile t
  __device__ __forceinline__ int operator()(int t) const { return raw(t) & ~1; }
  // whether tile t is part of a partial tile whose element bits apply
  __device__ __forceinline__ bool partial(int t) const { return (raw(t) & 1) != 0; }
  // list entry of tile t, and its sub-tile within that entry's block
  __device__ __forceinline__ int entry(int t) const { return e0 + t / sub; }
  __device__ __forceinline__ int sub_of(int t) const { return t - (t / sub) * sub; }
};

}  // namespace af
