// generic.h -- the strided / broadcast building blocks the unchanged autograd
// composes around the hot path: binary elementwise with broadcasting
// (vearo-backend-cpu elementwise_op, crates/vearo-backend-cpu/src/lib.rs:160-238),
// single-axis sum / mean (lib.rs:566-653), strided gather to contiguous (the
// device replacement for Tensor::contiguous, crates/vearo-core/src/tensor.rs:345-486)
// and a fill kernel (zeroing without hipMemset, so it is safe inside graphs).
#pragma once
#include "common.h"

VH_DEV float apply_op(int op, float a, float b) {
  switch (op) {
    case 0: return a + b;
    case 1: return a - b;
    case 2: return a * b;
    default: return a / b;
  }
}

// Offset of flat output index `i` under `l`'s strides, decomposed over `o`'s dims.
template <typename IT>
VH_DEV int64_t strided_offset(IT i, const StridedLayout& o, const StridedLayout& l) {
  int64_t off = 0;
  for (int d = o.rank - 1; d >= 0; --d) {
    const IT dim = (IT)o.dims[d];
    const IT c = i % dim;
    i /= dim;
    off += (int64_t)c * l.strides[d];
  }
  return off;
}

template <int VW>
VH_DEV void binary_contig_impl(const BinaryArgs& a) {
  const int64_t nu = a.n / VW;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < nu; u += stride) {
    const Unit<VW> l = load_stream<VW>(a.l + u * VW);
    const Unit<VW> r = load_stream<VW>(a.r + u * VW);
    Unit<VW> o;
#pragma unroll
    for (int j = 0; j < VW; ++j) o.v[j] = apply_op(a.op, l.v[j], r.v[j]);
    store_stream<VW>(a.out + u * VW, o);
  }
}

// op(full, vec) or op(vec, full) with a contiguous vector of length bn
// repeating along the rows of a contiguous full operand -- a bias add, the
// attention mask [S, S] added to [B, H, S, S] scores, or a single value (bn =
// 1: the unfused attention's scale): one unit per thread over the whole
// output, streaming loads and stores of the full operand, the vector read
// through the caches. VW divides bn (or bn = 1), so a unit stays within one row.
template <int VW>
VH_DEV void binary_rowbcast_impl(const BinaryArgs& a) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= a.n / VW) return;
  const float* full = a.vec_lhs ? a.r : a.l;
  const float* vec = a.vec_lhs ? a.l : a.r;
  const Unit<VW> f = load_stream<VW>(full + u * VW);
  Unit<VW> v;
  if (a.bn == 1) {
    const float s = vec[0];
#pragma unroll
    for (int j = 0; j < VW; ++j) v.v[j] = s;
  } else {
    v = *reinterpret_cast<const Unit<VW>*>(vec + (u * VW) % a.bn);
  }
  Unit<VW> o;
#pragma unroll
  for (int j = 0; j < VW; ++j) o.v[j] = a.vec_lhs ? apply_op(a.op, v.v[j], f.v[j]) : apply_op(a.op, f.v[j], v.v[j]);
  store_stream<VW>(a.out + u * VW, o);
}

// op(full, vec) or op(vec, full) with each vector element repeating over bn
// consecutive output elements (the vector spans the output's leading dims,
// with size-1 trailing dims: the Softmax arm's dy - sum(dy * y, keep_dim)).
// One unit per thread; VW divides bn, so a unit uses one vector element.
template <int VW>
VH_DEV void binary_colbcast_impl(const BinaryArgs& a) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= a.n / VW) return;
  const float* full = a.vec_lhs ? a.r : a.l;
  const float* vec = a.vec_lhs ? a.l : a.r;
  const Unit<VW> f = load_stream<VW>(full + u * VW);
  const float s = vec[(u * VW) / a.bn];
  Unit<VW> o;
#pragma unroll
  for (int j = 0; j < VW; ++j) o.v[j] = a.vec_lhs ? apply_op(a.op, s, f.v[j]) : apply_op(a.op, f.v[j], s);
  store_stream<VW>(a.out + u * VW, o);
}

template <typename IT>
VH_DEV void binary_strided_impl(const BinaryArgs& a) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
    const float l = a.l[strided_offset<IT>((IT)i, a.ol, a.ll)];
    const float r = a.r[strided_offset<IT>((IT)i, a.ol, a.rl)];
    a.out[i] = apply_op(a.op, l, r);
  }
}

// One thread per output; the reduced axis is walked in index order, which is the
// CPU's accumulation order for each output element (bit-exact).
VH_DEV void reduce_thread_impl(const ReduceArgs& a) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < a.n_out; o += stride) {
    const float* p = a.x + strided_offset<int64_t>(o, a.ol, a.ol);
    float s = 0.0f;
    for (int64_t k = 0; k < a.red_len; ++k) s += p[k * a.red_stride];
    a.out[o] = a.mean ? s / (float)a.red_len : s;
  }
}

// One wave per output for a unit-stride reduced axis (coalesced); per-lane
// sequential partials then a fixed wave tree.
VH_DEV void reduce_wave_impl(const ReduceArgs& a) {
  const int lane = threadIdx.x & 63;
  const int64_t o = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (o >= a.n_out) return;
  const float* p = a.x + strided_offset<int64_t>(o, a.ol, a.ol);
  float s = 0.0f;
  for (int64_t k = lane; k < a.red_len; k += 64) s += p[k];
  s = group_sum<64>(s);
  if (lane == 0) a.out[o] = a.mean ? s / (float)a.red_len : s;
}

template <typename IT>
VH_DEV void strided_copy_impl(const CopyArgs& a) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride)
    a.dst[i] = a.src[strided_offset<IT>((IT)i, a.sl, a.sl)];
}

// A transposed view made contiguous through a 64 x 64 LDS tile: reads run
// along the source's unit-stride dim (r), writes along the destination's (c),
// both 256 bytes per wave instruction; the tile is padded to 65 columns so
// the column reads hit 64 different banks.
VH_DEV void transpose_impl(const TransposeArgs& a) {
  __shared__ float t[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 64;
  const int64_t b = blockIdx.z;
  const float* src = a.src + (b / a.nb1) * a.sb0 + (b % a.nb1) * a.sb1;
  float* dst = a.dst + b * a.R * a.C;
  const int64_t r = r0 + tx;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t c = c0 + ty + 4 * i;
    if (r < a.R && c < a.C) t[ty + 4 * i][tx] = src[r + c * a.sc];
  }
  __syncthreads();
  const int64_t c = c0 + tx;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t rr = r0 + ty + 4 * i;
    if (rr < a.R && c < a.C) dst[rr * a.C + c] = t[tx][ty + 4 * i];
  }
}

// transpose_impl with 128-bit accesses on both sides: a thread loads 4
// consecutive r of one c and stores 4 consecutive c of one r. The host takes
// it when R, C and every stride are multiples of 4 and both bases are 16-byte
// aligned, so each 4-run is wholly inside or outside the matrix. LDS t[c][r]
// with a 65-float row: the writes (4 r of one c per thread) and the reads (one
// r of 4 c per thread) each hit 64 distinct banks per wave.
VH_DEV void transpose4_impl(const TransposeArgs& a) {
  __shared__ float t[64][65];
  const int q = threadIdx.x & 15, p = threadIdx.x >> 4;
  const int64_t c0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 64;
  const int64_t b = blockIdx.z;
  const float* src = a.src + (b / a.nb1) * a.sb0 + (b % a.nb1) * a.sb1;
  float* dst = a.dst + b * a.R * a.C;
  const int64_t r = r0 + 4 * q;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t c = c0 + p + 16 * i;
    if (r < a.R && c < a.C) {
      const float4 v = *reinterpret_cast<const float4*>(src + r + c * a.sc);
      float* row = &t[p + 16 * i][4 * q];
      row[0] = v.x; row[1] = v.y; row[2] = v.z; row[3] = v.w;
    }
  }
  __syncthreads();
  const int64_t c = c0 + 4 * q;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rl = p + 16 * i;
    const int64_t rr = r0 + rl;
    if (rr < a.R && c < a.C)
      *reinterpret_cast<float4*>(dst + rr * a.C + c) =
          make_float4(t[4 * q][rl], t[4 * q + 1][rl], t[4 * q + 2][rl], t[4 * q + 3][rl]);
  }
}

// The device's expf / logf / tanhf as the kernels call them (softmax's and
// cross-entropy's exp, cross-entropy's log, GELU's tanh): same functions,
// same build flags, one element per thread.
VH_DEV void math_probe_impl(const MathProbeArgs& a) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
    const float v = a.x[i];
    a.y[i] = a.fn == 0 ? expf(v) : a.fn == 1 ? logf(v) : tanhf(v);
  }
}

VH_DEV void fill_impl(const FillArgs& a) {
  const int64_t n4 = (reinterpret_cast<uintptr_t>(a.p) & 15) ? 0 : a.n / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const float v = a.value;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t u = tid; u < n4; u += stride)
    *reinterpret_cast<float4*>(a.p + u * 4) = make_float4(v, v, v, v);
  for (int64_t i = n4 * 4 + tid; i < a.n; i += stride) a.p[i] = v;
}

// dst = src, one 16-byte unit per thread, streaming loads and stores: one
// unit per thread and a grid over the whole buffer copy 768 MB at 6.4 TB/s
// on this GPU, against 5.3 TB/s for the runtime's copy kernel and 4.8-5.2
// for grid-striding forms (measured).
VH_DEV void stream_copy_impl(const StreamCopyArgs& a) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u < a.n4) store_stream<4>(a.dst + u * 4, load_stream<4>(a.src + u * 4));
}

// Column sums of rows [g*rpb, (g+1)*rpb) of x[rows, C]: part[g][c], summed in
// row order. Grid (G, ceil(C/256)); one thread per column, consecutive threads
// on consecutive columns (coalesced rows), 8 row loads in flight.
VH_DEV void col_partial_impl(const ColPartialArgs& a) {
  const int64_t c = (int64_t)blockIdx.y * 256 + threadIdx.x;
  if (c >= a.C) return;
  const int64_t r0 = (int64_t)blockIdx.x * a.rpb;
  const int64_t r1 = r0 + a.rpb < a.rows ? r0 + a.rpb : a.rows;
  const float* p = a.x + c;
  float s = 0.0f;
  int64_t r = r0;
  for (; r + 8 <= r1; r += 8) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = p[(r + k) * a.C];
#pragma unroll
    for (int k = 0; k < 8; ++k) s += v[k];
  }
  for (; r < r1; ++r) s += p[r * a.C];
  a.part[(int64_t)blockIdx.x * a.C + c] = s;
}

// One pass over an attention call's mask and operands. Grid (ceil(S / 16),
// 5 * Y): grid y = segment * Y + the leading (b, h) pair; a workgroup takes 16
// consecutive rows of one [.., S, last] block, 16 lanes to a row (128-bit
// loads when the row is contiguous and 16-byte aligned). Mask element
// (i, j) of its last two dims: j <= i must be +-0 (else flag 1); j > i must be
// <= -1 and not NaN (else flag 2), and the smallest |value| of those is
// tracked. q, k, v, g: the largest |x| as bits (NaN and inf sort above every
// finite value). The workgroup folds its lanes, then adds to slot
// (blockIdx.x + blockIdx.y) % 64 of `words` (8 words a slot: [0] flags (or),
// [1] 0x7f800000 - min |masked| bits (max), [2 + seg - 1] max |x| bits (max)),
// so no one address takes more than about a thousand atomics; the host folds the
// 64 slots. Integer or / max only: the result does not depend on timing.
VH_DEV void attn_probe_impl(const AttnProbeArgs& a) {
  __shared__ uint32_t red[3][4];
  const int seg = (int)(blockIdx.y / a.Y);
  const int32_t bh = (int32_t)(blockIdx.y % a.Y);
  const float* t = a.t[seg];
  const int32_t d1 = a.d1[seg], d2 = a.d2[seg], d3 = a.d3[seg];
  if (!t || bh >= a.d0[seg] * d1) return;
  const int l16 = threadIdx.x & 15;
  const float* blk = t + (int64_t)(bh / d1) * a.s0[seg] + (int64_t)(bh % d1) * a.s1[seg];
  const int64_t s2 = a.s2[seg], s3 = a.s3[seg];
  uint32_t hi = 0, lo = 0, bad = 0;  // lo: 0x7f800000 - |masked value| bits, largest kept
  auto see = [&](float x, int32_t j, int32_t i2) {
    const uint32_t m = __float_as_uint(x) & 0x7fffffffu;
    if (seg == 0) {
      if (j <= i2) {
        if (m != 0) bad |= 1u;
      } else if (!(x <= -1.0f)) {
        bad |= 2u;
      } else {
        const uint32_t c = 0x7f800000u - m;  // m <= 0x7f800000 here (NaN fails above)
        lo = c > lo ? c : lo;
      }
    } else {
      hi = m > hi ? m : hi;
    }
  };
  const int32_t i2 = (int32_t)blockIdx.x * 16 + (int32_t)(threadIdx.x >> 4);
  if (i2 < d2) {
    const float* row = blk + (int64_t)i2 * s2;
    if (s3 == 1 && d3 % 4 == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
#pragma unroll 4
      for (int32_t j = 4 * l16; j < d3; j += 64) {
        const float4 x = *reinterpret_cast<const float4*>(row + j);
        see(x.x, j, i2);
        see(x.y, j + 1, i2);
        see(x.z, j + 2, i2);
        see(x.w, j + 3, i2);
      }
    } else {
#pragma unroll 4
      for (int32_t j = l16; j < d3; j += 16) see(row[j * s3], j, i2);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t h2 = (uint32_t)__shfl_xor((int)hi, off, 64), l2 = (uint32_t)__shfl_xor((int)lo, off, 64);
    hi = h2 > hi ? h2 : hi;
    lo = l2 > lo ? l2 : lo;
    bad |= (uint32_t)__shfl_xor((int)bad, off, 64);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = bad;
    red[1][w] = lo;
    red[2][w] = hi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 4; ++i) {
      bad |= red[0][i];
      lo = red[1][i] > lo ? red[1][i] : lo;
      hi = red[2][i] > hi ? red[2][i] : hi;
    }
    uint32_t* slot = a.words + 8 * ((blockIdx.x + blockIdx.y) % 64);
    if (seg == 0) {
      if (bad) atomicOr(slot, bad);
      if (lo) atomicMax(slot + 1, lo);
    } else if (hi) {
      atomicMax(slot + 1 + seg, hi);
    }
  }
}

// The probe's verdict, one wave: fold the 64 slots (or of the flags, max of
// the rest), then the conditions under which skipping the masked blocks gives
// the dense masked form's bits, in double precision: no flagged mask entry
// and finite operands; a masked entry's x - rowmax below -256 with margin
// (|m|min (1 - 2^-22) - 2 smax (1 + 2^-22) > 256, smax the largest |score|
// scale * Dk * max|q| * max|k| widened by the f32 bound for a sum of Dk
// products, gamma = Dk u / (1 - Dk u), and the scaling's rounding), where f32
// exp is exactly 0; and, backward, Dk max|v| max|dO| < 1e37 so the products
// that meet those zeros stay finite. *flag = 1 then, else 0.
VH_DEV void attn_decide_impl(const AttnDecideArgs& a) {
  const int lane = threadIdx.x & 63;
  const uint32_t* w = a.words + 8 * lane;
  uint32_t h[6];
  h[0] = w[0];
#pragma unroll
  for (int j = 1; j < 6; ++j) h[j] = w[j];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    h[0] |= (uint32_t)__shfl_xor((int)h[0], off, 64);
#pragma unroll
    for (int j = 1; j < 6; ++j) {
      const uint32_t o = (uint32_t)__shfl_xor((int)h[j], off, 64);
      h[j] = o > h[j] ? o : h[j];
    }
  }
  if (lane != 0) return;
  auto fl = [](uint32_t b) { return (double)__uint_as_float(b); };
  const uint32_t kInf = 0x7f800000u;
  int ok = h[0] == 0u;  // an allowed entry not +-0, or a masked one above -1 or NaN
  ok = ok && h[2] < kInf && h[3] < kInf && h[4] < kInf && (!a.has_g || h[5] < kInf);  // NaN or inf
  const double u = 0x1p-24, nu = (double)a.Dk * u;
  ok = ok && nu < 0.25;
  if (ok) {
    const double smax = a.scale * (double)a.Dk * fl(h[2]) * fl(h[3]) * (1.0 + 2.0 * nu / (1.0 - nu)) * (1.0 + 2.0 * u);
    const double mmin = fl(kInf - h[1]);  // the smallest |masked value| (inf when there is none)
    ok = mmin * (1.0 - 0x1p-22) - 2.0 * smax * (1.0 + 0x1p-22) > 256.0;
    if (ok && a.has_g) ok = (double)a.Dk * fl(h[4]) * fl(h[5]) < 1e37;
  }
  *a.flag = ok ? 1 : 0;
}
