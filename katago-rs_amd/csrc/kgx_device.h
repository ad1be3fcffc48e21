// Device-side helpers shared by the kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <cfloat>
#include <stdexcept>
#include <string>
#include <type_traits>

#include "kgx_kernels.h"

namespace kgx {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));  // 16-byte staging (registers, unlike HIP's uint4 struct)

#define KGX_CHECK_LAUNCH()                                                                                    \
  do {                                                                                                        \
    hipError_t e_ = hipGetLastError();                                                                        \
    if (e_ != hipSuccess) throw std::runtime_error(std::string("kernel launch: ") + hipGetErrorString(e_)); \
  } while (0)

// Launches kernel k like k<<<grid, block, lds, s>>>(args...). While a profiled forward times its ops
// (g_launch_timing set), the launch goes through hipExtLaunchKernel, whose dispatch records the events around the
// kernel itself: the first kernel of an op records `start`, every kernel records `stop`, so an op's time spans its
// kernels and excludes the host-side launch latency in front of them.
template <typename... KArgs, typename... Args>
inline void launch_k(void (*k)(KArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
  LaunchTiming& t = g_launch_timing;
  if (t.start) {
    hipExtLaunchKernelGGL(k, grid, block, (std::uint32_t)lds, s, t.used ? nullptr : t.start, t.stop, 0u,
                          static_cast<KArgs>(args)...);
    t.used = true;
  } else {
    k<<<grid, block, lds, s>>>(static_cast<KArgs>(args)...);
  }
}

template <int ACT>
__device__ __forceinline__ float act_f(float a) {
  if constexpr (ACT == ACT_RELU) {
    return fmaxf(a, 0.f);
  } else if constexpr (ACT == ACT_MISH) {
    // a * tanh(softplus(a)); with e = exp(a), tanh(log(1 + e)) = e (e + 2) / (e (e + 2) + 2). Softplus is the
    // identity above 20 (burn's threshold), where tanh is 1 in float. Branch-free: the exponent is clamped so
    // that n stays finite, and the select picks the identity.
    const float e = __expf(fminf(a, 20.f));
    const float n = e * (e + 2.f);
    const float r = a * n * __builtin_amdgcn_rcpf(n + 2.f);
    return a > 20.f ? a : r;
  } else if constexpr (ACT == ACT_SILU) {
    return a * __builtin_amdgcn_rcpf(__expf(-a) + 1.f);  // x / (exp(-x) + 1)
  } else {
    return a;
  }
}

// The activation chosen at run time (uniform across a launch).
__device__ __forceinline__ float act_rt(float a, int kind) {
  switch (kind) {
    case ACT_RELU: return act_f<ACT_RELU>(a);
    case ACT_MISH: return act_f<ACT_MISH>(a);
    case ACT_SILU: return act_f<ACT_SILU>(a);
    default: return a;
  }
}

// act(a) * mk for a value stored as a 16-bit operand with no low plane. Mish is the same function as act_f's,
// written as b - 2 b q with b = a * mk, q = 1 / (e (e + 2) + 2), e = exp(a): eight instructions where act_f's form
// and the mask take thirteen. It needs no clamp or select: a large a gives e = inf, q = 0 and the result b. For
// negative a the difference cancels, an absolute error of a few float ulps of a, far below the 16-bit rounding that
// follows. The result is pinned as a float (an empty asm), so that no kernel fuses the last multiply-add into the
// conversion to 16 bits: one rounding there instead of two would make kernels that emit the same activation differ
// in the last bit.
template <int ACT>
__device__ __forceinline__ float act16(float a, float mk) {
  if constexpr (ACT == ACT_MISH) {
    const float e = __expf(a);
    const float q = __builtin_amdgcn_rcpf(__builtin_fmaf(e, e + 2.f, 2.f));
    const float b = a * mk;
    float r = __builtin_fmaf(-2.f * b, q, b);
    asm("" : "+v"(r));
    return r;
  } else {
    return act_f<ACT>(a) * mk;
  }
}
__device__ __forceinline__ float act16_rt(float a, int kind, float mk) {
  switch (kind) {
    case ACT_RELU: return act16<ACT_RELU>(a, mk);
    case ACT_MISH: return act16<ACT_MISH>(a, mk);
    case ACT_SILU: return act16<ACT_SILU>(a, mk);
    default: return a * mk;
  }
}

template <typename T>
__device__ __forceinline__ T to_t(float v) { return (T)v; }

template <typename T> struct Tile;
template <> struct Tile<float> { static constexpr int VEC = 4; };
template <> struct Tile<f16> { static constexpr int VEC = 8; };
template <> struct Tile<bf16> { static constexpr int VEC = 8; };

// 16x16 MFMA over one 16-byte K slice of T operands: f16/bf16 K = 32 (v_mfma_f32_16x16x32_*), float K = 4
// (v_mfma_f32_16x16x4_f32, called four times per 16 bytes by the callers).
template <typename T>
__device__ __forceinline__ floatx4 mfma16(const T* a, const T* b, floatx4 c) {
  if constexpr (std::is_same<T, f16>::value) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8*)a, *(const half8*)b, c, 0, 0, 0);
  } else if constexpr (std::is_same<T, bf16>::value) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8*)a, *(const bf16x8*)b, c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(*a, *b, c, 0, 0, 0);
  }
}

// The conv / GEMM epilogue for one output element (row m, column n) with its accumulated value: bias, board mask,
// compute-type store, float store (or residual add) and emission of the consumer's activation.
template <typename T>
__device__ __forceinline__ void conv_store(const ConvOut& o, int m, int n, float v) {
  if (o.colbias) v += o.colbias[(size_t)(m / HW) * o.ld_colbias + n];
  if (o.rowmask) v *= o.rowmask[m];
  if (o.yt) ((T*)o.yt)[(size_t)m * o.ldyt + n] = to_t<T>(v);
  if (o.y) {
    float* p = o.y + (size_t)m * o.ldy + n;
    if (o.accumulate) v += *p;
    if (!o.y_dead) *p = v;
  }
  if (o.emit.scale) {
    const float x = v * o.emit.scale[n] + o.emit.bias[n];
    const float a = sizeof(T) == 2 && !o.emit.out_lo ? act16_rt(x, o.emit.act, o.emit.mask[m])
                                                     : act_rt(x, o.emit.act) * o.emit.mask[m];
    const T hi = to_t<T>(a);
    ((T*)o.emit.out)[(size_t)m * o.emit.ld + n] = hi;
    if (o.emit.out_lo) ((T*)o.emit.out_lo)[(size_t)m * o.emit.ld + n] = to_t<T>(a - (float)hi);
  }
}

// Epilogue for four consecutive channels n..n+3 of pixel m (conv_store on a float4). The per-pixel inputs come
// preloaded: the residual `yacc` (when o.accumulate), the row mask `rm`, the emit scale/bias `es`/`eb` of the
// four channels and the emit mask `mk` (the epilogue's stores may alias them as far as the compiler knows, so a
// load placed between stores would wait a full round trip). The column bias (the stem's global input bias, one
// launch per forward) is read inline.
// Four consecutive compute-type values in one store (8 bytes for 16-bit types, 16 for float).
template <typename T>
__device__ __forceinline__ void store4(T* p, float a, float b, float c, float d) {
  if constexpr (sizeof(T) == 4) {
    *(floatx4*)p = floatx4{a, b, c, d};
  } else {
    T t[4] = {to_t<T>(a), to_t<T>(b), to_t<T>(c), to_t<T>(d)};
    *(uint2*)p = *(const uint2*)t;
  }
}

// The outputs a ConvOut asks for, as a bit set (store_flags): known to a caller that specializes conv_store4 on
// them, so that the store path has no branch.
enum StoreFlags {
  SF_COLBIAS = 1, SF_ROWMASK = 2, SF_YT = 4, SF_Y = 8, SF_ACC = 16, SF_YDEAD = 32, SF_EMIT = 64, SF_LO = 128
};
__host__ __device__ inline int store_flags(const ConvOut& o) {
  return (o.colbias ? SF_COLBIAS : 0) | (o.rowmask ? SF_ROWMASK : 0) | (o.yt ? SF_YT : 0) | (o.y ? SF_Y : 0) |
         (o.y && o.accumulate ? SF_ACC : 0) | (o.y && o.y_dead ? SF_YDEAD : 0) | (o.emit.scale ? SF_EMIT : 0) |
         (o.emit.scale && o.emit.out_lo ? SF_LO : 0);
}

// ACT >= 0: the emission's activation, known to the caller (o.emit.act); -1: chosen here at run time. FL >= 0:
// store_flags(o), known to the caller; -1: read from o here.
template <typename T, int ACT = -1, int FL = -1>
__device__ __forceinline__ void conv_store4(const ConvOut& o, int m, int n, floatx4 v, floatx4 yacc, float rm,
                                            floatx4 es, floatx4 eb, float mk) {
  const int fl = FL >= 0 ? FL : store_flags(o);
  if (fl & SF_COLBIAS) v += *(const floatx4*)(o.colbias + (size_t)(m / HW) * o.ld_colbias + n);
  if (fl & SF_ROWMASK) v *= rm;
  if (fl & SF_YT) store4<T>((T*)o.yt + (size_t)m * o.ldyt + n, v[0], v[1], v[2], v[3]);
  if (fl & SF_Y) {
    if (fl & SF_ACC) v += yacc;
    // Non-temporal: the float stream's next reader is a later op (the next residual add, two or more launches
    // on), so its lines go out to MALL instead of taking L2 from the activations and weights of the ops between.
    if (!(fl & SF_YDEAD)) __builtin_nontemporal_store(v, (floatx4*)(o.y + (size_t)m * o.ldy + n));
  }
  if (fl & SF_EMIT) {
    float t[4];
    // (16-bit operands without a low plane take act16's form.)
    const bool h16 = sizeof(T) == 2 && !(fl & SF_LO);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float a = v[e] * es[e] + eb[e];
      if constexpr (ACT >= 0) t[e] = h16 ? act16<ACT>(a, mk) : act_f<ACT>(a) * mk;
      else t[e] = h16 ? act16_rt(a, o.emit.act, mk) : act_rt(a, o.emit.act) * mk;
    }
    store4<T>((T*)o.emit.out + (size_t)m * o.emit.ld + n, t[0], t[1], t[2], t[3]);
    if (fl & SF_LO) {
      // Split operands: the low part is what the 16-bit high part leaves of the float activation (exact in float).
      float l[4];
#pragma unroll
      for (int e = 0; e < 4; e++) l[e] = t[e] - (float)to_t<T>(t[e]);
      store4<T>((T*)o.emit.out_lo + (size_t)m * o.emit.ld + n, l[0], l[1], l[2], l[3]);
    }
  }
}

// One 16-byte-per-lane load straight into LDS (buffer_load ... lds): lane i's bytes [off, off + 16) of the
// range [base, base + nbytes) land at lds + 16 i; offsets past the range read as zero. The buffer resource is
// built here so that kernels never hold its type.
__device__ __forceinline__ void lds_load16(const void* base, int nbytes, void* lds, int off) {
  typedef __attribute__((address_space(3))) void* lds_ptr_t;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(__builtin_amdgcn_make_buffer_rsrc((void*)base, 0, nbytes, 0x00020000),
                                           (lds_ptr_t)lds, 16, off, 0, 0, 0);
}

// Touches this workgroup's share of the 128-byte lines of [p, p + nbytes), so that they are in its XCD's L2 when the
// next launch reads them: workgroup g runs on XCD g mod 8, and the n workgroups of that XCD take lines s + n t (s =
// g / 8) for thread t, one 4-byte buffer load each (so a launch covers up to n x threads lines per XCD; offsets past
// the range read as zero without a memory access, so a null range touches nothing). The kernel keeps the returned
// value live up to its end (l2_touch_keep), which it reaches on every path: the load is not dropped, and no wait
// for it comes before that point.
__device__ __forceinline__ int l2_touch(const char* p, int nbytes, int tid) {
  const int v = __builtin_amdgcn_raw_buffer_load_b32(__builtin_amdgcn_make_buffer_rsrc((void*)p, 0, nbytes, 0x00020000),
                                                     l2_touch_line(blockIdx.x, gridDim.x, tid) * 128, 0, 0);
  asm volatile("" ::: "memory");  // issued here, not next to its use
  return v;
}
__device__ __forceinline__ void l2_touch_keep(int v) { asm volatile("" ::"v"(v)); }

// Winograd F(TM x TM, 3x3) geometry on the 19x19 board.
template <int TM>
struct Wino {
  static constexpr int TI = TM + 2;               // input tile side
  static constexpr int NP = TI * TI;              // tile points = batched GEMMs
  static constexpr int TX = (POS + TM - 1) / TM;  // tiles per board side
  static constexpr int NT = TX * TX;              // tiles per board
};

}  // namespace kgx
