// Streaming fused dequant-GEMV + low-rank correction (gfx950, group 128).
//
// Same result as gemv_tile (glq_gemv_core.h) for 1 <= M <= 16, built for HBM
// bandwidth instead of simplicity:
//  * Row-split: each wave owns whole 16-row tiles (full K), so it never waits
//    on another wave after the one-time staging of x and a.
//  * Codes, scales and zero-points reach LDS by direct global->LDS loads
//    (global_load_lds_dwordx4 / _dword), so the data in flight occupies no
//    VGPRs.  Each wave keeps a ring of D chunk slots; a chunk is 16 rows x
//    128 contiguous bytes of every row (2 load instructions of 8 rows x 128 B,
//    the pattern the MI355X memory system serves fastest) plus the chunk's
//    scales and zero-points.  D-1 chunks are in flight while one is consumed,
//    across tile boundaries.
//  * The 16-byte pieces of a chunk are permuted across lanes (piece ^ (row/2))
//    so the MFMA-layout reads from LDS are bank-conflict free.
//  * MFMA roles: A = x (token rows), B = codes (weight rows as columns), so
//    D[token][row] and each lane needs one scale and one zero-point per step.
//    2-bit steps (256 codes, two 128-code groups) keep their two groups apart
//    inside one MFMA: group-half h's x goes to A rows 8h..8h+7 (zeros
//    elsewhere), so D rows 0-7 / 8-15 are the two half sums; tokens 8..15 take
//    a second pass; halves merge with one cross-lane add per tile.
//  * The compiler does not order LDS reads after direct-to-LDS loads, so the
//    kernel waits explicitly: before consuming chunk c it waits until at most
//    NI*(D-1) vector-memory operations are outstanding, where NI is the number
//    of load instructions per chunk.  Loads of one wave complete in order, and
//    any store or ordinary load issued after chunk c's loads only makes that
//    wait stricter, so chunk c is in LDS when the wait returns.  Before a
//    slot is refilled, all LDS reads of the wave have completed (lgkmcnt(0)).
#pragma once

#include "glq_gemv_core.h"

namespace glq {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kStreamCodeBytes = 2048;  // 16 rows x 128 B
constexpr int kStreamSzBytes = 512;     // scales + zero-points of a chunk (dword per lane)
constexpr int kStreamSlot = kStreamCodeBytes + kStreamSzBytes;

// Explicit waits.  Inline asm with a memory clobber, so no compiler pass moves
// an LDS access across them.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Shape/layout of a streaming launch (every item has the same K and N).
struct StreamShape {
  int K, N, G, rank, rpad, sym, kw;
  int svb;         // bytes of one SV/bias buffer (32*rank rounded up to 1 KiB, + 256)
  int nsv;         // SV/bias buffers per wave (tiles whose SV may be in flight)
  int nchunk;      // 128-byte chunks per row (last one may be partial)
  int tiles;       // 16-row tiles per item
  int xstride;     // halves per staged token row of x
  int mmax;        // largest M of any item
  int apad;        // halves per token row of staged a
};

struct StreamLds {
  int xs, xc, a, ring, total;  // byte offsets; xc = [chunk128][16 tokens] x 2 floats
};

// x rows are padded to a multiple of 256 codes (zeros), plus one all-zero
// row that masked lanes read; the per-chunk sums get matching zero padding.
__host__ __device__ inline int stream_kpad(int K) { return (K + 255) / 256 * 256; }

template <int D>
__host__ __device__ inline StreamLds stream_lds(int mmax, int K, int xstride, int apad, int svb,
                                                int nsv) {
  StreamLds L;
  int o = 0;
  L.xs = o;   o += al16((mmax + 1) * xstride * 2);
  L.xc = o;   o += al16((stream_kpad(K) / 128) * 32 * 4);
  L.a = o;    o += al16(16 * apad * 2);
  L.ring = o; o += 4 * (D * kStreamSlot + nsv * svb);
  L.total = o;
  return L;
}

// Issues the direct-to-LDS loads of a tile's SV rows (16 x rank fp16,
// contiguous in memory, dwordx4 per lane) and bias (16 fp16, dword per lane).
__device__ __forceinline__ void stream_issue_sv(const __half* SV, const __half* B,
                                                const StreamShape& sh, int r0,
                                                unsigned char* buf, int lane) {
  const int rowbytes = sh.rank * 2;
  const int nbytes = SV ? 16 * rowbytes : 0;
  for (int I = 0; I * 1024 < nbytes; ++I) {
    const int o = I * 1024 + 16 * lane;  // byte offset within the 16-row block
    const int row = min(o, nbytes - 16) / rowbytes;
    const int col = min(o, nbytes - 16) - row * rowbytes;
    const char* src = (const char*)SV + (int64_t)min(r0 + row, sh.N - 1) * rowbytes + col;
    __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(buf + I * 1024), 16, 0, 0);
  }
  if (B) {
    // dword q (< 8) holds bias[r0 + 2q], bias[r0 + 2q + 1] (N is even); past
    // the last row it re-reads the last dword, whose values are never stored
    const int n = min(r0 + 2 * (lane & 7), sh.N - 2);
    __builtin_amdgcn_global_load_lds((const void*)(B + n), (lds_void*)(buf + sh.svb - 256), 4, 0,
                                     0);
  }
}

// Element index (row n, group g) of a scale / zero-point, clamped in bounds.
__device__ __forceinline__ int64_t sz_index(const StreamShape& sh, int r, int g) {
  return (int64_t)min(r, sh.N - 1) * sh.G + min(g, sh.G - 1);
}

// Issues the direct-to-LDS loads of chunk `ch` of the tile at row r0: codes
// (2 x dwordx4: lane q of instruction I carries row 8I + q/8, 16-byte piece
// (q%8) ^ ((row/2)%8)), then the chunk's scales and zero-points as the
// aligned dwords that contain them (2-bit: lane q -> row q/4, group 4ch+q%4,
// one instruction each for s and z; 4-bit: lane q -> row (q%32)/2, group
// 2ch+q%2, s in lanes 0-31 and z in 32-63).  The host guarantees N*G is even,
// so every such dword lies inside the tensor.
template <int BITS>
__device__ __forceinline__ void stream_issue(const uint32_t* C, const __half* S, const __half* Z,
                                             const StreamShape& sh, int r0, int ch,
                                             unsigned char* slot, int lane) {
  const char* cb = (const char*)C;
  const int64_t rowbytes = (int64_t)sh.kw * 4;
  const int64_t total = rowbytes * sh.N;
#pragma unroll
  for (int I = 0; I < 2; ++I) {
    const int row = 8 * I + (lane >> 3);
    const int piece = (lane & 7) ^ ((row >> 1) & 7);
    const int n = min(r0 + row, sh.N - 1);
    int64_t off = (int64_t)n * rowbytes + 128 * ch + 16 * piece;
    if (off + 16 > total) off = total - 16;  // tail of the last row: stay in bounds
    __builtin_amdgcn_global_load_lds((const void*)(cb + off), (lds_void*)(slot + 1024 * I), 16,
                                     0, 0);
  }
  const __half* Zs = sh.sym ? S : Z;
  unsigned char* szs = slot + kStreamCodeBytes;
  if constexpr (BITS == 2) {
    const int64_t e = sz_index(sh, r0 + (lane >> 2), 4 * ch + (lane & 3));
    __builtin_amdgcn_global_load_lds((const void*)(S + (e & ~1ll)), (lds_void*)szs, 4, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(Zs + (e & ~1ll)), (lds_void*)(szs + 256), 4, 0,
                                     0);
  } else {
    const int q = lane & 31;
    const int64_t e = sz_index(sh, r0 + (q >> 1), 2 * ch + (q & 1));
    const __half* base = lane < 32 ? S : Zs;
    __builtin_amdgcn_global_load_lds((const void*)(base + (e & ~1ll)), (lds_void*)szs, 4, 0, 0);
  }
}

template <int BITS>
constexpr int stream_ni() { return BITS == 2 ? 4 : 3; }

// Per-lane constants of the consume loop (computed once per workgroup).
template <int MP>
struct StreamLane {
  int code_off[2];  // byte offset of this lane's 16 B of codes in a slot, per step
  int xa[MP];       // half offset of this lane's x operand row (or the zero row)
  int xcb[MP];      // float offset of this lane's c1 values in a 128-code chunk row
  int szb;          // byte offset of this lane's scale dword in a slot
  int h;            // 2-bit: group-half of this lane's D rows and codes
};

// Consumes one chunk (2 steps) of a tile from its LDS slot into yacc.
// Branch-free: masked lanes read the zero x row; a group past K (2-bit tail)
// gets scale 0; rowpar = parity of the tile row's first scale element.
template <int BITS, int MP, bool SYM>
__device__ __forceinline__ void stream_consume(const unsigned char* slot, int ch, int rowpar,
                                               const StreamShape& sh, const __half* xs,
                                               const float* xc, f32x4 (&yacc)[MP],
                                               const StreamLane<MP>& ln,
                                               const DecodeConsts& dk) {
  // symmetric codes are b-bit two's complement: flipping the top bit maps
  // them to q + 2^(b-1), whose zero-point is 2^(b-1)
  constexpr uint32_t xor_mask = SYM ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  const float zsym = (float)(1 << (BITS - 1));
  const unsigned char* sz = slot + kStreamCodeBytes;
#pragma unroll
  for (int sp = 0; sp < 2; ++sp) {
    u32x4 w = *(const u32x4*)(slot + ln.code_off[sp]);
    if constexpr (SYM) w ^= xor_mask;
    const int st = 2 * ch + sp;
    if constexpr (BITS == 2) {
      // scale / zero-point of group 4ch + 2sp + h: dword (row*4 + 2sp + h)
      const int c128 = 2 * st + ln.h;
      const int sh16 = 16 * (rowpar ^ ln.h);
      const uint32_t sw_ = *(const uint32_t*)(sz + ln.szb + 8 * sp);
      float s = __half2float(__ushort_as_half((uint16_t)(sw_ >> sh16)));
      s = c128 * 128 < sh.K ? s : 0.f;
      float z = zsym;
      if constexpr (!SYM) {
        const uint32_t zw = *(const uint32_t*)(sz + 256 + ln.szb + 8 * sp);
        z = __half2float(__ushort_as_half((uint16_t)(zw >> sh16)));
      }
      f32x4 acc[MP];
#pragma unroll
      for (int p = 0; p < MP; ++p) acc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f16x8 b0, b1;
        decode2(w[i], b0, b1, dk);
#pragma unroll
        for (int p = 0; p < MP; ++p) {
          const __half* xr = xs + ln.xa[p] + st * 256 + 16 * i;
          acc[p] = mfma_16x16x32(*(const f16x8*)xr, b0, acc[p]);
          acc[p] = mfma_16x16x32(*(const f16x8*)(xr + 8), b1, acc[p]);
        }
      }
#pragma unroll
      for (int p = 0; p < MP; ++p) {
        const f32x4 c1 = *(const f32x4*)(xc + c128 * 32 + ln.xcb[p]);
        const f32x4 c2 = *(const f32x4*)(xc + c128 * 32 + 16 + ln.xcb[p]);
#pragma unroll
        for (int i = 0; i < 4; ++i) yacc[p][i] += s * (acc[p][i] - fmaf(z, c2[i], c1[i]));
      }
    } else {
      const int sh16 = 16 * (rowpar ^ sp);
      const uint32_t sw_ = *(const uint32_t*)(sz + ln.szb + 4 * sp);
      float s = __half2float(__ushort_as_half((uint16_t)(sw_ >> sh16)));
      s = st * 128 < sh.K ? s : 0.f;
      float z = zsym;
      if constexpr (!SYM) {
        const uint32_t zw = *(const uint32_t*)(sz + 128 + ln.szb + 4 * sp);
        z = __half2float(__ushort_as_half((uint16_t)(zw >> sh16)));
      }
      const __half* xr = xs + ln.xa[0] + st * 128;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc = mfma_16x16x32(*(const f16x8*)(xr + 8 * i), decode4(w[i], dk), acc);
      const f32x4 c1 = *(const f32x4*)(xc + st * 32 + ln.xcb[0]);
      const f32x4 c2 = *(const f32x4*)(xc + st * 32 + 16 + ln.xcb[0]);
#pragma unroll
      for (int i = 0; i < 4; ++i) yacc[0][i] += s * (acc[i] - fmaf(z, c2[i], c1[i]));
    }
  }
}

// One workgroup: tiles [t0, t1) of one item; wave w takes t0 + w, t0 + w + 4, ...
template <int BITS, int MP, int D, bool SYM, class Src>
__device__ void gemv_stream(const Src& src, const StreamShape& sh, int item, int t0, int t1,
                            unsigned char* smem) {
  constexpr int NI = stream_ni<BITS>();
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  const int M = src.m_rows(item);
  const StreamLds L = stream_lds<D>(sh.mmax, sh.K, sh.xstride, sh.apad, sh.svb, sh.nsv);
  __half* xs = (__half*)(smem + L.xs);  // (mmax + 1) rows; row mmax is all zero
  float* xc = (float*)(smem + L.xc);    // [c128][c1 x16 | c2 x16]
  __half* a_l = (__half*)(smem + L.a);
  unsigned char* ring = smem + L.ring + wave * (D * kStreamSlot + sh.nsv * sh.svb);
  unsigned char* svbuf = ring + D * kStreamSlot;  // nsv buffers of SV rows + bias

  const uint32_t* C = src.codes(item);
  const __half* S = src.scales(item);
  const __half* Z = src.zeros(item);
  const __half* SV = src.sv(item);
  const __half* B = src.bias(item);
  const bool lora = sh.rank > 0 && SV != nullptr;
  const bool per_tile = lora || B != nullptr;

  // This wave's work list: tiles t0 + wave + 4j, nchunk chunks each.
  const int ntile_w = t1 - t0 > wave ? (t1 - t0 - wave + 3) / 4 : 0;
  const int total = ntile_w * sh.nchunk;
  auto issue = [&](int un) {
    const int ch = un % sh.nchunk;
    const int j = un / sh.nchunk;
    const int r0 = (t0 + wave + 4 * j) * 16;
    if (ch == 0 && per_tile)
      stream_issue_sv(lora ? SV : nullptr, B, sh, r0, svbuf + (j % sh.nsv) * sh.svb, lane);
    stream_issue<BITS>(C, S, Z, sh, r0, ch, ring + (un % D) * kStreamSlot, lane);
  };

  // ---- prologue: D-1 chunks in flight, then stage x, its sums, and a ----
  for (int u = 0; u < D - 1 && u < total; ++u) issue(u);

  const int kpad = stream_kpad(sh.K);
  {
    const int nb = kpad >> 4;  // 16-code blocks per padded token row
    const int totalb = (sh.mmax + 1) * nb;
    for (int base = 0; base < totalb; base += 256) {
      const int idx = base + tid;
      const bool v = idx < totalb;
      float s = 0.f, sb = 0.f;
      int m = 0, blk = 0;
      if (v) {
        m = idx / nb;
        blk = idx - m * nb;
        _Float16 in[16], o[16];
        if (m < M && blk * 16 < sh.K) {
          const f16x8* srcx = (const f16x8*)(src.xrow(item, m) + blk * 16);
          const f16x8 in0 = srcx[0], in1 = srcx[1];
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            in[c] = in0[c];
            in[8 + c] = in1[c];
          }
        } else {
#pragma unroll
          for (int c = 0; c < 16; ++c) in[c] = (_Float16)0.f;
        }
#pragma unroll
        for (int pos = 0; pos < 16; ++pos) {
          o[pos] = in[perm_src<BITS>(pos)];
          const float f = (float)o[pos];
          s += f;
          sb += code_bias<BITS>(pos) * f;
        }
        f16x8 o0, o1;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          o0[c] = o[c];
          o1[c] = o[8 + c];
        }
        f16x8* dst = (f16x8*)(xs + m * sh.xstride + blk * 16);
        dst[0] = o0;
        dst[1] = o1;
      }
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 4);
      sb += __shfl_xor(sb, 1);
      sb += __shfl_xor(sb, 2);
      sb += __shfl_xor(sb, 4);
      if (v && (idx & 7) == 0 && m < sh.mmax) {
        const int c128 = blk >> 3;
        xc[c128 * 32 + m] = sb;      // c1: sum of operand bias * x
        xc[c128 * 32 + 16 + m] = s;  // c2: sum of x
      }
    }
    // tokens mmax..15 of every chunk read as zero
    const int nc = kpad >> 7, nz = 16 - sh.mmax;
    for (int idx = tid; idx < nc * nz; idx += 256) {
      const int c128 = idx / nz, m = sh.mmax + idx % nz;
      xc[c128 * 32 + m] = 0.f;
      xc[c128 * 32 + 16 + m] = 0.f;
    }
  }
  if (lora) {
    for (int idx = tid; idx < 16 * sh.rpad; idx += 256) {
      const int m = idx / sh.rpad, j = idx - m * sh.rpad;
      a_l[m * sh.apad + j] =
          (m < M && j < sh.rank) ? src.load_a(item, m, j) : __float2half(0.f);
    }
  }
  __syncthreads();

  // ---- per-lane constants ----
  StreamLane<MP> ln;
  {
    const int sw = (li >> 1) & 7;
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) ln.code_off[sp] = li * 128 + (((4 * sp + kb) ^ sw) << 4);
    const int zrow = sh.mmax * sh.xstride;
    if constexpr (BITS == 2) {
      ln.h = kb >> 1;
#pragma unroll
      for (int p = 0; p < MP; ++p) {
        const int m = (li & 7) + 8 * p;
        const bool act = ((li >> 3) == ln.h) && m < M;
        ln.xa[p] = (act ? m * sh.xstride : zrow) + 64 * kb;
        ln.xcb[p] = 8 * p + 4 * (kb & 1);
      }
      ln.szb = 4 * (li * 4 + ln.h);
    } else {
      ln.h = 0;
      ln.xa[0] = (li < M ? li * sh.xstride : zrow) + 32 * kb;
      ln.xcb[0] = 4 * kb;
      ln.szb = 8 * li;
    }
  }

  // ---- stream: consume chunk u while chunks u+1 .. u+D-1 are in flight ----
  const DecodeConsts dk = DecodeConsts::make();
  f32x4 yacc[MP];
#pragma unroll
  for (int p = 0; p < MP; ++p) yacc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
  int ch = 0, jt = 0, slot = 0;
  int r0 = (t0 + wave) * 16;
  int rowpar = (int)(((int64_t)min(r0 + li, sh.N - 1) * sh.G) & 1);
  for (int u = 0; u < total; ++u) {
    if (u + D - 1 < total) {
      wait_lgkm0();  // slot (u-1)%D: every LDS read of it has completed
      issue(u + D - 1);
      wait_vmcnt<NI * (D - 1)>();
    } else {
      wait_vmcnt<0>();
    }
    stream_consume<BITS, MP, SYM>(ring + slot * kStreamSlot, ch, rowpar, sh, xs, xc, yacc, ln,
                                  dk);
    if (++slot == D) slot = 0;
    if (++ch == sh.nchunk) {
      // ---- tile epilogue (this wave only); its SV rows and bias arrived
      //      with the tile's first chunk ----
      const unsigned char* sb = svbuf + (jt % sh.nsv) * sh.svb;
      f32x4 y;
      if constexpr (BITS == 2) {
        f32x4 y0 = yacc[0], y1 = yacc[MP - 1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          y0[i] += __shfl_xor(y0[i], 32);
          if (MP == 2) y1[i] += __shfl_xor(y1[i], 32);
        }
        y = kb < 2 ? y0 : (MP == 2 ? y1 : f32x4{0.f, 0.f, 0.f, 0.f});
      } else {
        y = yacc[0];
      }
      if (lora) {
        const __half* svr = (const __half*)sb + li * sh.rank;
        for (int s = 0; s < sh.rpad; s += 32) {
          const int j = s + 8 * kb;
          const f16x8 bv = j < sh.rank ? *(const f16x8*)(svr + j) : f16x8{};
          const f16x8 av = *(const f16x8*)(a_l + li * sh.apad + j);
          y = mfma_16x16x32(av, bv, y);
        }
      }
      const int n = r0 + li;
      if (n < sh.N) {
        const float bn = B ? __half2float(((const __half*)(sb + sh.svb - 256))[li]) : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 4 * kb + i;
          if (m < M) src.store(item, m, n, y[i] + bn);
        }
      }
#pragma unroll
      for (int p = 0; p < MP; ++p) yacc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
      ch = 0;
      ++jt;
      r0 += 64;
      rowpar = (int)(((int64_t)min(r0 + li, sh.N - 1) * sh.G) & 1);
    }
  }
}

}  // namespace glq
