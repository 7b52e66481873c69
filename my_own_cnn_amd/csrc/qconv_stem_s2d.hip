// int8 convolution for stride-2 thin-channel stems (c <= 4, e.g. the ResNet 7x7/2 stem with
// c = 3) as a stride-1 convolution over a space-to-depth copy of the input built in LDS.
//
// Space to depth.  S2D pixel (I, J) holds the 2 x 2 input pixels (2I + a - ph, 2J + b - pw),
// a, b in {0, 1}, c bytes each, in the order (a, b, channel), zero-padded to 16 bytes (one
// MFMA chunk).  Output pixel (ho, wo) then reads the ceil(r/2) x ceil(s/2) s2d pixels
// (ho + u, wo + v): tap (u, v) is one 16-byte chunk whose byte (2a + b)*c + ch meets filter
// element (2u + a, 2v + b, ch), zero where 2u + a >= r or 2v + b >= s.  The reduction has
// T = ceil(r/2) * ceil(s/2) chunks, KB = ceil(T/4) K-blocks of v_mfma_i32_16x16x64_i8 (the
// 7x7 stem: 16 chunks, 4 K-blocks), and every MFMA operand is one aligned 16-byte LDS read:
// lane (rho, g) of K-block kb reads chunk q = 4kb + g at s2d pixel (ho + q / V, wo0 + rho +
// q % V).  Consecutive lanes read consecutive s2d pixels of one row, which the LDS serves
// without bank conflicts (lanes that meet read the same address).
//
// Work.  A workgroup of 8 waves owns a band of BH output rows of one image and 64 output
// channels.  It loads the band's 2 * (BH + ceil(r/2) - 1) input rows (global -> LDS DMA,
// 1 KB per instruction, zeros outside the image) and the 64 channels' filter bytes, then
// builds the s2d rows and the filter chunks (operand slots, swizzled so that every fragment
// read is free of bank conflicts) with VALU work once per byte, and keeps the filter
// fragments in registers.  Each wave then takes 16-pixel segments of the band's output rows
// in turn; the matrix instructions of the next segment are issued before the requantization
// of the current one (mma_requant_pipe4 for the 16-chunk filters), so the two overlap.  The
// output stage is the other int8 kernels' (bias as the first MFMA's C operand; convert,
// scale, clamp, round; one 16-byte store of 16 consecutive channels per lane, followed by
// store_gap()).

#include "qconv_device.h"

#include <algorithm>
#include <atomic>

namespace miq {
namespace {

constexpr int kSdWaves = 8;
constexpr int kSdLds = 160 * 1024;
constexpr int kSdPitch = 2048;  // bytes per staged s2d row: up to 128 s2d pixels

struct S2dArgs {
  const int8_t* x;
  const int8_t* w;
  const int32_t* bias;   // int8 outputs: bias; Q32: the filter row sums T (offset codes)
  const float* wscale;   // int8 outputs: scales; Q32: the per-image records {dx, dw, Kdim * dx * dw, 0}
  void* y;               // int8, or int32 for Q32
  int H, W, C, K, R, S, Ho, Wo, ph, pw;
  int V, T;             // s2d taps per row (ceil(s/2)) and in all (ceil(r/2) * V)
  int BH, bands_per_img, nbands, nblocks, SEGR;
  int P, PLB, rows_ld;  // staged input row pitch (a multiple of 1 KB), its left pad, loads per row
  int HS, ncols;        // s2d rows per band and s2d columns built per row
  int RSC, nfilt;       // filter bytes per channel, filter load instructions
  int filt_lds, ep_lds, slot_lds, raw_lds, s2d_lds;
  float act_scale;
  FastDivM fd_nbands, fd_bpi, fd_segr, fd_rowsld, fd_npairs;
};

static_assert(sizeof(S2dArgs) <= 256, "kernel arguments fit one s_load batch");

// 8 bytes of an LDS byte array from byte o (any alignment), as two dwords.
__device__ __forceinline__ unsigned long long lds_bytes8(const unsigned char* base, int o) {
  const unsigned* p = reinterpret_cast<const unsigned*>(base + (o & ~3));
  const unsigned sh = static_cast<unsigned>(o & 3);
  const unsigned d0 = p[0], d1 = p[1], d2 = p[2];
  const unsigned lo = __builtin_amdgcn_alignbyte(d1, d0, sh);
  const unsigned hi = __builtin_amdgcn_alignbyte(d2, d1, sh);
  return static_cast<unsigned long long>(lo) | (static_cast<unsigned long long>(hi) << 32);
}

// Filter chunk q of channel kl sits at 16-byte slot 16 kl + ((q + 2 kl + 8 (kl / 16)) mod 16).  A
// ds_read_b128 serves 16 lanes per cycle: one half-wave's lane quads 4i .. 4i + 3 whose quad
// index i has one popcount parity.  In both channel orders of the fragments (int8 outputs and
// int32 outputs) those 16 lanes read 16 distinct slots modulo 16, so the fragment reads are free
// of bank conflicts.
__device__ __forceinline__ int s2d_slot(int kl, int q) { return 16 * kl + ((q + 2 * kl + 8 * (kl >> 4)) & 15); }

// 16 bytes to LDS byte address addr, issued by inline assembly: the compiler puts a wait for
// all of the wave's outstanding global -> LDS loads in front of any LDS store it emits (it
// cannot tell the loads' LDS destinations apart), and the filter chunks are written while the
// input rows are still loading.  The caller waits for lgkmcnt(0) before the barrier that
// publishes the stores.
__device__ __forceinline__ void sd_lds_store16(unsigned addr, v4i v) {
  asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(v) : "memory");
}

// 2C bytes (C <= 4) from byte o of an LDS byte array (any alignment), in the low bytes.
template <int C>
__device__ __forceinline__ unsigned long long lds_pair(const unsigned char* base, int o) {
  constexpr unsigned long long keep = C == 4 ? ~0ull : ((1ull << (16 * C)) - 1ull);
  return lds_bytes8(base, o) & keep;
}

// One 16-byte chunk from two 2C-byte pieces: bytes [0, 2C) from lo, [2C, 4C) from hi, zeros
// after.
template <int C>
__device__ __forceinline__ v4i s2d_chunk(unsigned long long lo, unsigned long long hi) {
  unsigned long long w0, w1;
  if constexpr (C == 4) {
    w0 = lo;
    w1 = hi;
  } else {
    w0 = lo | (hi << (16 * C));
    w1 = hi >> (64 - 16 * C);
  }
  return v4i{static_cast<int>(w0), static_cast<int>(w0 >> 32), static_cast<int>(w1), static_cast<int>(w1 >> 32)};
}

// The 64 channels' filter chunks: chunk q = tap (u, v) = (q / V, q % V), for a = 0, 1 the 2C
// bytes of filter row 2u + a, columns 2v and 2v + 1 (contiguous in KRSC); a column 2v + 1 = s
// or a row 2u + a >= r contributes zeros; chunks past T are zero.
template <int C, int FR, int FS>
__device__ __forceinline__ void s2d_filter(const S2dArgs& a, const unsigned char* bytes, unsigned base, int tid) {
  const int R = FR ? FR : a.R;
  const int S = FS ? FS : a.S;
  const int V = FS ? (FS + 1) / 2 : a.V;
  const int T = FR ? ((FR + 1) / 2) * V : a.T;
  const unsigned char* fb = bytes + a.filt_lds;
  const unsigned slots = base + static_cast<unsigned>(a.slot_lds);
  const int rowc = S * C;  // bytes of one filter row
  for (int idx = tid; idx < 64 * 16; idx += 64 * kSdWaves) {
    const int kl = idx >> 4;
    const int q = idx & 15;
    unsigned long long piece[2] = {0ull, 0ull};
    if (q < T) {
      const int u = q / V;
      const int v = q - u * V;
      // the second column of the pair exists unless 2v + 1 == s
      const unsigned long long keep = 2 * v + 1 < S ? ~0ull : ((1ull << (8 * C)) - 1ull);
#pragma unroll
      for (int r2 = 0; r2 < 2; ++r2) {
        const int r = 2 * u + r2;
        if (r < R) piece[r2] = lds_pair<C>(fb, kl * (R * rowc) + r * rowc + 2 * v * C) & keep;
      }
    }
    sd_lds_store16(slots + 16u * static_cast<unsigned>(s2d_slot(kl, q)), s2d_chunk<C>(piece[0], piece[1]));
  }
}

// The 7x7 three-channel filter's chunks, a thread per (channel kl, tap row u) = (t / 4, t % 4):
// filter rows 2u and 2u + 1 (21 bytes each; row 7 does not exist) read as seven aligned
// dwords each, their column pairs v = 0 .. 3 (6 bytes at 6v; v = 3 holds column 6 only) the
// chunks (u, v).  A ds_write_b128 stores 8 consecutive lanes per cycle (128 bytes, measured:
// its bank conflicts follow slot mod 8 over those lanes, unlike the reads).  The thread writes
// chunk (v + lane / 2 + 2 (lane / 4)) mod 4 in its v-th store, which puts every 8 consecutive
// lanes on 8 distinct slots modulo 8.
__device__ __forceinline__ void s2d_filter_773(const S2dArgs& a, const unsigned char* bytes, unsigned base, int tid) {
  const unsigned* fw = reinterpret_cast<const unsigned*>(bytes + a.filt_lds);
  const unsigned slots = base + static_cast<unsigned>(a.slot_lds);
  const int rot = (tid >> 1) + 2 * (tid >> 2);
  for (int t = tid; t < 64 * 4; t += 64 * kSdWaves) {
    const int kl = t >> 2;
    const int u = t & 3;
    unsigned long long pc[2][4];
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2) {
      const int r = 2 * u + r2;
#pragma unroll
      for (int v = 0; v < 4; ++v) pc[r2][v] = 0ull;
      if (r < 7) {
        const int s0 = kl * 147 + r * 21;
        const unsigned* p = fw + (s0 >> 2);
        const unsigned sh = static_cast<unsigned>(s0 & 3);
        unsigned w[7];
#pragma unroll
        for (int k = 0; k < 7; ++k) w[k] = p[k];
        unsigned al[6];
#pragma unroll
        for (int k = 0; k < 6; ++k) al[k] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], sh);
        const unsigned long long w01 = al[0] | (static_cast<unsigned long long>(al[1]) << 32);
        const unsigned long long w23 = al[2] | (static_cast<unsigned long long>(al[3]) << 32);
        const unsigned long long w45 = al[4] | (static_cast<unsigned long long>(al[5]) << 32);
        constexpr unsigned long long k6 = (1ull << 48) - 1ull;
        pc[r2][0] = w01 & k6;                             // bytes 0 .. 5
        pc[r2][1] = ((w01 >> 48) | (w23 << 16)) & k6;     // bytes 6 .. 11
        pc[r2][2] = ((w23 >> 32) | (w45 << 32)) & k6;     // bytes 12 .. 17
        pc[r2][3] = (w45 >> 16) & ((1ull << 24) - 1ull);  // bytes 18 .. 20 (column 6)
      }
    }
    v4i ch[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) ch[v] = s2d_chunk<3>(pc[0][v], pc[1][v]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int vv = (v + rot) & 3;
      const v4i c01 = (vv & 1) ? ch[1] : ch[0];
      const v4i c23 = (vv & 1) ? ch[3] : ch[2];
      sd_lds_store16(slots + 16u * static_cast<unsigned>(s2d_slot(kl, 4 * u + vv)), (vv & 2) ? c23 : c01);
    }
  }
}

// The 4C bytes of an s2d pixel pair (2m, 2m + 1) in one staged row, from the four dwords at
// and after its first byte's dword (sh = that byte's offset inside it): the first pixel's 2C
// bytes in p0, the second's in p1.
template <int C>
__device__ __forceinline__ void s2d_pair_pieces(const unsigned (&w)[4], unsigned sh, unsigned long long& p0,
                                                unsigned long long& p1) {
  const unsigned a0 = __builtin_amdgcn_alignbyte(w[1], w[0], sh);
  const unsigned a1 = __builtin_amdgcn_alignbyte(w[2], w[1], sh);
  const unsigned a2 = __builtin_amdgcn_alignbyte(w[3], w[2], sh);
  const unsigned long long lo = static_cast<unsigned long long>(a0) | (static_cast<unsigned long long>(a1) << 32);
  if constexpr (C == 4) {
    // 4C = 16 bytes: the pair starts on a dword (PLB and pw C = 4 pw are multiples of 4), sh = 0
    p0 = lo;
    p1 = static_cast<unsigned long long>(w[2]) | (static_cast<unsigned long long>(w[3]) << 32);
  } else {
    constexpr unsigned long long keep = (1ull << (16 * C)) - 1ull;
    const unsigned long long hi = static_cast<unsigned long long>(a2);
    p0 = lo & keep;
    p1 = ((lo >> (16 * C)) | (hi << (64 - 16 * C))) & keep;
  }
}

// The band's s2d rows: pixel (I, J) from staged input rows 2I and 2I + 1, 2C bytes each at
// byte PLB + (2J - pw) * C.  A thread builds pixel pairs (2m, 2m + 1): the pair's 4C bytes of a
// row start at a byte offset sh = (PLB - pw C) mod 4 that is the same for every pair, so each
// row is read as four aligned dwords, consecutive lanes 12 bytes apart (distinct banks).  Lanes
// 4 .. 7 of every 8 write the pair's second chunk first, so the 8 consecutive lanes of each
// ds_write_b128 cycle meet 8 distinct slots modulo 8.  Two pairs per thread and pass, their reads issued before
// their writes.  A pair past the last column (ncols odd) writes the unused slot ncols.
template <int C>
__device__ __forceinline__ void s2d_rows(const S2dArgs& a, const unsigned char* bytes, v4i* lds, int tid) {
  constexpr int kU = 2;
  const unsigned* raw = reinterpret_cast<const unsigned*>(bytes + a.raw_lds);
  const int npairs = (a.ncols + 1) >> 1;
  const int total = a.HS * npairs;
  const int o0 = a.PLB - a.pw * C;  // >= 0: PLB is pw * C rounded up to 16
  const unsigned sh = static_cast<unsigned>(o0 & 3);
  for (int idx0 = tid; idx0 < total; idx0 += kU * 64 * kSdWaves) {
    unsigned w0[kU][4], w1[kU][4];
    int dst[kU];
#pragma unroll
    for (int e = 0; e < kU; ++e) {
      const int idx = min(idx0 + e * 64 * kSdWaves, total - 1);  // repeats the last pair past the end
      const int I = fdiv(idx, a.fd_npairs);
      const int m = idx - I * npairs;
      const int d = (o0 + 4 * m * C) >> 2;
      const unsigned* r0 = raw + (2 * I) * (a.P >> 2) + d;
      const unsigned* r1 = r0 + (a.P >> 2);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        w0[e][k] = r0[k];
        w1[e][k] = r1[k];
      }
      dst[e] = (a.s2d_lds + I * kSdPitch) / 16 + 2 * m;
    }
#pragma unroll
    for (int e = 0; e < kU; ++e) {
      unsigned long long x0, x1, y0, y1;
      s2d_pair_pieces<C>(w0[e], sh, x0, x1);
      s2d_pair_pieces<C>(w1[e], sh, y0, y1);
      const v4i c0 = s2d_chunk<C>(x0, y0);
      const v4i c1 = s2d_chunk<C>(x1, y1);
      const bool sw = (tid >> 2) & 1;
      lds[dst[e] + (sw ? 1 : 0)] = sw ? c1 : c0;
      lds[dst[e] + (sw ? 0 : 1)] = sw ? c0 : c1;
    }
  }
}

// FC, FR, FS: the channel count and filter size when fixed at compile time (the 7x7 stem with
// three channels), 0 where they come from the arguments.
// This lane's window-sum mask of K-block kb: 0x01 at the bytes of its chunk q = 4kb + g (tap
// (u, v) = (q / V, q % V)) that meet a filter element: byte (2a + b) * C + ch with
// 2u + a < R, 2v + b < S, ch < C; zero for chunks past T.
__device__ __forceinline__ v4i s2d_window_mask(int R, int S, int C, int V, int T, int kb, int g) {
  const int q = 4 * kb + g;
  const int u = q / V;
  const int v = q - u * V;
  v4i m = {0, 0, 0, 0};
  if (q < T) {
#pragma unroll
    for (int byte = 0; byte < 16; ++byte) {
      const int pc = byte / C;   // pixel (2a + b) of the 2 x 2 block
      const int ab = pc < 4 ? pc : 4;
      const bool ok = ab < 4 && 2 * u + (ab >> 1) < R && 2 * v + (ab & 1) < S;
      if (ok) m[byte >> 2] |= 1 << (8 * (byte & 3));
    }
  }
  return m;
}

// Q32: the int32 route of the reference's float-code API on offset codes (x' = code - o on an
// image padded with zx - o, w' = code - o): accumulators start at dx * T(k) + Kdim * dx * dw,
// each lane sums its chunks' input bytes under s2d_window_mask (v_dot4), the 4 lanes of a
// pixel add theirs to the window sum W(p), and the store adds dw * W(p); outputs are int32 in
// natural channel order (MFMA row block j, row rho <-> channel 16j + rho), so the 4 lanes of a
// pixel write 64 contiguous bytes per instruction.
template <int KB, bool RELU, int FC, int FR, int FS, bool Q32>
__global__ void __launch_bounds__(64 * kSdWaves, 1) i8_stem_s2d_kernel(S2dArgs a_in) {
  const S2dArgs a = preload_args(a_in);
  extern __shared__ v4i sd_lds[];
  const unsigned char* bytes = reinterpret_cast<const unsigned char*>(sd_lds);
  const unsigned base = static_cast<unsigned>(reinterpret_cast<uintptr_t>(sd_lds) & 0xffffffffu);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rho = lane & 15;
  const int g = lane >> 4;

  const int lin = xcd_tile(blockIdx.x, a.nblocks);
  const int ctile = fdiv(lin, a.fd_nbands);
  const int band = lin - ctile * a.nbands;
  const int n = fdiv(band, a.fd_bpi);
  const int bi = band - n * a.bands_per_img;
  const int k0 = ctile * 64;
  const int ho0 = bi * a.BH;
  const int band_rows = min(a.BH, a.Ho - ho0);

  // ---- loads: filter instruction f (bytes [1024f + 16l, +16) of the tile's 64 * RSC
  // contiguous KRSC bytes) and input instruction i = row * rows_ld + m go to wave f % 8 and
  // i % 8; bias and scales to wave 0.  Input row rr of the band is image row 2*ho0 - ph + rr;
  // staged row byte PLB + b holds row byte b (zeros outside the image).
  {
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + static_cast<size_t>(k0) * a.RSC, 64 * a.RSC);
    for (int f = wave; f < a.nfilt; f += kSdWaves)
      load_lds16(rw, sd_lds + a.filt_lds / 16 + f * 64, 16u * lane, 1024u * f);
  }
  if (wave == 0) {
    load_lds16(make_rsrc(a.bias ? a.bias + k0 : nullptr, a.bias ? 256 : 0), sd_lds + a.ep_lds / 16, 16u * lane, 0);
    if constexpr (Q32) {
      load_lds16(make_rsrc(a.wscale + 4 * static_cast<size_t>(n), 16), sd_lds + a.ep_lds / 16 + 64, 16u * lane, 0);
    } else {
      load_lds16(make_rsrc(a.wscale + k0, 256), sd_lds + a.ep_lds / 16 + 64, 16u * lane, 0);
    }
  }
  const int ni = 2 * a.HS * a.rows_ld;
  {
    const int rowb = a.W * a.C;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + static_cast<size_t>(n) * a.H * rowb, a.H * rowb);
    const int hi0 = 2 * ho0 - a.ph;
    for (int i = wave; i < ni; i += kSdWaves) {
      const int rr = fdiv(i, a.fd_rowsld);
      const int m = i - rr * a.rows_ld;
      const int hi = hi0 + rr;
      const int b = 1024 * m + 16 * lane - a.PLB;
      const unsigned soff =
          static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) ? static_cast<unsigned>(hi * rowb) : 0x40000000u;
      const unsigned voff = (b >= 0 && b + 16 <= rowb) ? static_cast<unsigned>(b) : 0x40000000u;
      load_lds16(rx, sd_lds + a.raw_lds / 16 + i * 64, voff, soff);
    }
  }
  // ---- the filter and parameter loads (issued before the rows, and loads complete in order)
  // have landed once this wave has at most its row loads outstanding; the filter chunks and
  // the fragments' register copy then overlap the input rows' loads ----
  wait_vmcnt(ni > wave ? (ni - wave + kSdWaves - 1) / kSdWaves : 0);
  barrier_only();
  if constexpr (FC != 0) {
    if constexpr (FC == 3 && FR == 7 && FS == 7) {
      s2d_filter_773(a, bytes, base, tid);
    } else {
      s2d_filter<FC, FR, FS>(a, bytes, base, tid);
    }
  } else {
    switch (a.C) {
      case 1: s2d_filter<1, 0, 0>(a, bytes, base, tid); break;
      case 2: s2d_filter<2, 0, 0>(a, bytes, base, tid); break;
      case 3: s2d_filter<3, 0, 0>(a, bytes, base, tid); break;
      default: s2d_filter<4, 0, 0>(a, bytes, base, tid); break;
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  barrier_only();

  // filter fragments: A[kb][j], lane (rho, g) = channel 16*(rho/4) + 4j + rho%4 (Q32: 16j +
  // rho), chunk 4kb + g
  v4i A[KB][4];
  {
    const v4i* slots = sd_lds + a.slot_lds / 16;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        A[kb][j] = slots[s2d_slot(Q32 ? 16 * j + rho : 16 * (rho >> 2) + 4 * j + (rho & 3), 4 * kb + g)];
  }
  // bias and requantization multipliers of the lane's channels k0 + 16g + 4j + i; Q32: the
  // accumulator start dx * T + Kdim * dx * dw of channels k0 + 16j + 4g + i
  v4i bias_v[4];
  v4f mult_v[4];
  unsigned qdw = 0;
  if constexpr (Q32) {
    const v4i rec = sd_lds[a.ep_lds / 16 + 64];
    const unsigned dx = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(rec[0]));
    qdw = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(rec[1]));
    const unsigned c0 = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(rec[2]));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4i tv = sd_lds[a.ep_lds / 16 + 4 * j + g];
#pragma unroll
      for (int i = 0; i < 4; ++i) bias_v[j][i] = static_cast<int>(dx * static_cast<unsigned>(tv[i]) + c0);
      mult_v[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bias_v[j] = sd_lds[a.ep_lds / 16 + 4 * g + j];
      const v4i ws = sd_lds[a.ep_lds / 16 + 64 + 4 * g + j];
#pragma unroll
      for (int i = 0; i < 4; ++i) mult_v[j][i] = requant_multiplier(a.act_scale, __int_as_float(ws[i]));
    }
  }
  // ---- the input rows have landed: the s2d rows ----
  wait_vmcnt(0);
  barrier_only();
  if constexpr (FC != 0) {
    s2d_rows<FC>(a, bytes, sd_lds, tid);
  } else {
    switch (a.C) {
      case 1: s2d_rows<1>(a, bytes, sd_lds, tid); break;
      case 2: s2d_rows<2>(a, bytes, sd_lds, tid); break;
      case 3: s2d_rows<3>(a, bytes, sd_lds, tid); break;
      default: s2d_rows<4>(a, bytes, sd_lds, tid); break;
    }
  }
  __syncthreads();
  // this lane's B chunk of K-block kb within a segment: s2d row offset u * pitch, column
  // rho + v (chunks past T read tap T - 1, whose filter chunk is zero)
  unsigned boff[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int V = FS ? (FS + 1) / 2 : a.V;
    const int T = FR ? ((FR + 1) / 2) * V : a.T;
    const int q = min(4 * kb + g, T - 1);
    const int u = q / V;
    const int v = q - u * V;
    boff[kb] = base + static_cast<unsigned>(a.s2d_lds + u * kSdPitch + 16 * (rho + v));
  }
  constexpr int kOutBytes = Q32 ? 4 : 1;
  const size_t out0 = (static_cast<size_t>(n) * a.Ho + ho0) * a.Wo * a.K + k0;
  const __amdgpu_buffer_rsrc_t ry =
      make_rsrc(static_cast<char*>(a.y) + out0 * kOutBytes, band_rows * a.Wo * a.K * kOutBytes);
  const int nseg = band_rows * a.SEGR;

  auto seg_b = [&](int sg, v4i (&B)[KB]) {
    const int t = fdiv(sg, a.fd_segr);
    const int wo0 = 16 * (sg - t * a.SEGR);
    const unsigned so = static_cast<unsigned>(t * kSdPitch + 16 * wo0);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) B[kb] = lds_read16(boff[kb] + so);
  };
  // a pixel past the row's end gets an offset 2^30 higher: past num_records, dropped
  auto out_voff = [&](int sg, int ch) {
    const int t = fdiv(sg, a.fd_segr);
    const int wo = 16 * (sg - t * a.SEGR) + rho;
    return static_cast<unsigned>(((t * a.Wo + wo) * a.K + ch) * kOutBytes) + (static_cast<unsigned>(wo >= a.Wo) << 30);
  };
  int sg = wave;
  if constexpr (Q32) {
    // window-sum masks of this lane's chunks
    v4i wm[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      wm[kb] = s2d_window_mask(FR ? FR : a.R, FS ? FS : a.S, FC ? FC : a.C, FS ? (FS + 1) / 2 : a.V,
                               FR ? ((FR + 1) / 2) * ((FS + 1) / 2) : a.T, kb, g);
    }
    auto mma_seg = [&](const v4i (&B)[KB], v4i (&acc)[4], int& ws) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0][j], B[0], bias_v[j], 0, 0, 0);
#pragma unroll
      for (int kb = 1; kb < KB; ++kb)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[kb][j], B[kb], acc[j], 0, 0, 0);
      // the dwords that hold input bytes (4C of 16; the rest of a chunk is zero)
      constexpr int kDw = FC ? (4 * FC + 3) / 4 : 4;
      ws = 0;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int d = 0; d < kDw; ++d) ws = __builtin_amdgcn_sdot4(B[kb][d], wm[kb][d], ws, false);
    };
    auto store32 = [&](int sg_, const v4i (&acc)[4], int ws) {
      ws += __shfl_xor(ws, 16);
      ws += __shfl_xor(ws, 32);
      const unsigned corr = qdw * static_cast<unsigned>(ws);
      const unsigned vo = out_voff(sg_, 4 * g);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v4i v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = static_cast<int>(static_cast<unsigned>(acc[j][i]) + corr);
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, vo + 64u * j, 0, kStoreAux);
        store_gap(v);
      }
    };
    if (sg < nseg) {
      v4i acc[4];
      int ws;
      {
        v4i B[KB];
        seg_b(sg, B);
        mma_seg(B, acc, ws);
      }
      // the first segment is stored before the pipelined loop starts (stores bound the loop)
      if (sg + kSdWaves < nseg) {
        store32(sg, acc, ws);
        sg += kSdWaves;
        v4i B[KB];
        seg_b(sg, B);
        mma_seg(B, acc, ws);
      }
      for (;;) {
        const int sn = sg + kSdWaves;
        if (sn >= nseg) break;
        v4i B[KB], accn[4];
        int wsn;
        seg_b(sn, B);
        mma_seg(B, accn, wsn);
        store32(sg, acc, ws);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = accn[j];
        ws = wsn;
        sg = sn;
      }
      store32(sg, acc, ws);
    }
  } else {
    auto store = [&](int sg_, const unsigned (&pk)[4]) {
      const v4i pkv = {static_cast<int>(pk[0]), static_cast<int>(pk[1]), static_cast<int>(pk[2]),
                       static_cast<int>(pk[3])};
      __builtin_amdgcn_raw_buffer_store_b128(pkv, ry, out_voff(sg_, 16 * g), 0, kStoreAux);
      store_gap(pkv);
    };
    // Software-pipelined by one segment: each matrix instruction of the next segment is issued
    // with a share of this segment's output stage (mma_requant_steps), so the two overlap.
    if (sg < nseg) {
      v4i acc[4];
      {
        v4i B[KB];
        seg_b(sg, B);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0][j], B[0], bias_v[j], 0, 0, 0);
#pragma unroll
        for (int kb = 1; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[kb][j], B[kb], acc[j], 0, 0, 0);
      }
      // the first segment's output goes out before the pipelined loop starts: the stores are the
      // main loop's bound, and they start one segment earlier
      {
        const int sn = sg + kSdWaves;
        if (sn < nseg) {
          unsigned pk[4];
          float f[16];
          requant_values<0, 16>(acc, mult_v, RELU ? 0.0f : -128.0f, f, pk);
          store(sg, pk);
          sg = sn;
          v4i B[KB];
          seg_b(sg, B);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0][j], B[0], bias_v[j], 0, 0, 0);
#pragma unroll
          for (int kb = 1; kb < KB; ++kb)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[kb][j], B[kb], acc[j], 0, 0, 0);
        }
      }
      for (;;) {
        const int sn = sg + kSdWaves;
        if (sn >= nseg) break;
        v4i B[KB];
        seg_b(sn, B);
        v4i accn[4];
        unsigned pk[4];
        float f[16];
        if constexpr (KB == 4) {
          mma_requant_pipe4(A, B, bias_v, accn, acc, mult_v, RELU ? 0.0f : -128.0f, f, pk);
        } else {
          mma_requant_steps<KB>(A, B, bias_v, accn, acc, mult_v, RELU ? 0.0f : -128.0f, f, pk);
        }
        store(sg, pk);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = accn[j];
        sg = sn;
      }
      unsigned pk[4];
      float f[16];
      requant_values<0, 16>(acc, mult_v, RELU ? 0.0f : -128.0f, f, pk);
      store(sg, pk);
    }
  }
}

struct S2dPlan {
  int V, T, KB, BH, bands_per_img, HS, ncols, P, PLB, rows_ld, nfilt;
  int filt_lds, ep_lds, slot_lds, raw_lds, s2d_lds;
  size_t lds;
};

int sd_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

int sd_round_up(long long v, int m) { return static_cast<int>((v + m - 1) / m * m); }

bool sd_plan(const Geom& g, S2dPlan* p, std::string* why, int out_bytes = 1) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  if (g.G != 1) return no("s2d stem kernel needs groups == 1");
  if (g.sh != 2 || g.sw != 2) return no("s2d stem kernel needs stride 2");
  if (g.dh != 1 || g.dw != 1) return no("s2d stem kernel needs dilation 1");
  if (g.C < 1 || g.C > 4) return no("s2d stem kernel needs 1 <= c <= 4");
  if (g.ph < 0 || g.pw < 0 || g.R < 1 || g.S < 1) return no("s2d stem kernel needs a filter and padding >= 0");
  if (g.K % 64 != 0) return no("s2d stem kernel needs k % 64 == 0");
  p->V = (g.S + 1) / 2;
  p->T = ((g.R + 1) / 2) * p->V;
  if (p->T > 16) return no("s2d stem kernel needs ceil(r/2) * ceil(s/2) <= 16");
  p->KB = (p->T + 3) / 4;
  const long long rowb = static_cast<long long>(g.W) * g.C;
  if (rowb % 16 != 0) return no("s2d stem kernel needs w * c % 16 == 0");
  if (static_cast<long long>(g.H) * rowb >= (1LL << 30)) return no("s2d stem kernel needs images below 2^30 bytes");
  if (static_cast<long long>(g.Ho) * g.Wo * g.K * out_bytes >= (1LL << 30)) {
    return no("s2d stem kernel needs outputs below 2^30 bytes per image");
  }
  const int segr = (g.Wo + 15) / 16;
  p->ncols = 16 * segr + p->V - 1;
  if (p->ncols > kSdPitch / 16) return no("s2d stem kernel needs output width + ceil(s/2) <= 113");
  p->PLB = sd_round_up(static_cast<long long>(g.pw) * g.C, 16);
  // the end of the last row read: four dwords from the last pixel pair's first byte
  const long long last = p->PLB + (4LL * ((p->ncols + 1) / 2 - 1) - g.pw) * g.C + 16;
  p->P = sd_round_up(std::max<long long>(p->PLB + rowb, last), 1024);
  p->rows_ld = p->P / 1024;
  const long long RSC = static_cast<long long>(g.R) * g.S * g.C;
  p->nfilt = static_cast<int>((64 * RSC + 1023) / 1024);
  const int cus = sd_cu_count();
  // filter bytes, 2 KB of bias and scales, 16 KB of operand slots, then per band the staged
  // input rows and the s2d rows
  const size_t fixed = static_cast<size_t>(p->nfilt) * 1024 + 2048 + 16384;
  const int Ru = (g.R + 1) / 2;
  bool found = false;
  double best = 0.0;
  for (int bh = 1; bh <= g.Ho; ++bh) {
    const long long hs = bh + Ru - 1;
    const size_t lds = fixed + static_cast<size_t>(2 * hs) * p->P + static_cast<size_t>(hs) * kSdPitch;
    if (lds > static_cast<size_t>(kSdLds)) break;
    const long long bands = (g.Ho + bh - 1) / bh;
    const long long wgs = static_cast<long long>(g.N) * bands * (g.K / 64);
    const long long rounds = (wgs + cus - 1) / cus;
    const double cost = static_cast<double>(rounds) * ((bh * segr + kSdWaves - 1) / kSdWaves + 3);
    if (!found || cost < best - 1e-9) {
      found = true;
      best = cost;
      p->BH = bh;
      p->bands_per_img = static_cast<int>(bands);
      p->HS = static_cast<int>(hs);
      p->lds = lds;
    }
  }
  if (!found) return no("s2d stem kernel band does not fit in LDS");
  p->filt_lds = 0;
  p->ep_lds = p->nfilt * 1024;
  p->slot_lds = p->ep_lds + 2048;
  p->raw_lds = p->slot_lds + 16384;
  p->s2d_lds = p->raw_lds + 2 * p->HS * p->P;
  const long long blocks = static_cast<long long>(g.N) * p->bands_per_img * (g.K / 64);
  if (blocks > 0x7fffffffLL) return no("grid too large");
  return true;
}

bool sd_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool stem_s2d_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                       std::string* why) {
  if (epi != kEpiI8) {
    if (why) *why = "s2d stem kernel: int8 outputs only";
    return false;
  }
  if (!sd_aligned16(x) || !sd_aligned16(w) || !sd_aligned16(y) || !sd_aligned16(rq.wscale) ||
      (rq.bias && !sd_aligned16(rq.bias))) {
    if (why) *why = "s2d stem kernel needs 16-byte aligned x, w, y, bias and scales";
    return false;
  }
  S2dPlan pl;
  return sd_plan(g, &pl, why);
}

namespace {

S2dArgs sd_args(const Geom& g, const S2dPlan& pl, const int8_t* x, const int8_t* w, void* y, const int32_t* bias,
                const float* wscale, float act_scale) {
  S2dArgs a;
  a.x = x; a.w = w; a.bias = bias; a.wscale = wscale; a.y = y;
  a.H = g.H; a.W = g.W; a.C = g.C; a.K = g.K; a.R = g.R; a.S = g.S; a.Ho = g.Ho; a.Wo = g.Wo;
  a.ph = g.ph; a.pw = g.pw;
  a.V = pl.V; a.T = pl.T;
  a.BH = pl.BH; a.bands_per_img = pl.bands_per_img; a.nbands = g.N * pl.bands_per_img;
  a.nblocks = a.nbands * (g.K / 64);
  a.SEGR = (g.Wo + 15) / 16;
  a.P = pl.P; a.PLB = pl.PLB; a.rows_ld = pl.rows_ld;
  a.HS = pl.HS; a.ncols = pl.ncols;
  a.RSC = g.R * g.S * g.C; a.nfilt = pl.nfilt;
  a.filt_lds = pl.filt_lds; a.ep_lds = pl.ep_lds; a.slot_lds = pl.slot_lds; a.raw_lds = pl.raw_lds;
  a.s2d_lds = pl.s2d_lds;
  a.act_scale = act_scale;
  a.fd_nbands = fastdiv_m(a.nbands);
  a.fd_bpi = fastdiv_m(pl.bands_per_img);
  a.fd_segr = fastdiv_m(a.SEGR);
  a.fd_rowsld = fastdiv_m(pl.rows_ld);
  a.fd_npairs = fastdiv_m((pl.ncols + 1) / 2);
  return a;
}

template <typename Kern>
void sd_go(Kern kern, const S2dArgs& a, const S2dPlan& pl, hipStream_t stream) {
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(pl.lds));
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(a.nblocks)), dim3(64 * kSdWaves), pl.lds, stream, a);
}

}  // namespace

hipError_t launch_i8_stem_s2d(const Geom& g, const int8_t* x, const int8_t* w, int8_t* y, const Requant& rq,
                              hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  S2dPlan pl;
  if (!sd_plan(g, &pl, nullptr)) return hipErrorInvalidConfiguration;
  const S2dArgs a = sd_args(g, pl, x, w, y, rq.bias, rq.wscale, rq.act_scale);
  const bool relu = rq.relu != 0;
  if (g.C == 3 && g.R == 7 && g.S == 7) {
    relu ? sd_go(i8_stem_s2d_kernel<4, true, 3, 7, 7, false>, a, pl, stream)
         : sd_go(i8_stem_s2d_kernel<4, false, 3, 7, 7, false>, a, pl, stream);
  } else {
    switch (pl.KB) {
      case 1: relu ? sd_go(i8_stem_s2d_kernel<1, true, 0, 0, 0, false>, a, pl, stream)
                   : sd_go(i8_stem_s2d_kernel<1, false, 0, 0, 0, false>, a, pl, stream); break;
      case 2: relu ? sd_go(i8_stem_s2d_kernel<2, true, 0, 0, 0, false>, a, pl, stream)
                   : sd_go(i8_stem_s2d_kernel<2, false, 0, 0, 0, false>, a, pl, stream); break;
      case 3: relu ? sd_go(i8_stem_s2d_kernel<3, true, 0, 0, 0, false>, a, pl, stream)
                   : sd_go(i8_stem_s2d_kernel<3, false, 0, 0, 0, false>, a, pl, stream); break;
      default: relu ? sd_go(i8_stem_s2d_kernel<4, true, 0, 0, 0, false>, a, pl, stream)
                    : sd_go(i8_stem_s2d_kernel<4, false, 0, 0, 0, false>, a, pl, stream); break;
    }
  }
  return hipGetLastError();
}

bool stem_s2d_qi32_plan_ok(const Geom& g, std::string* why) {
  S2dPlan pl;
  return sd_plan(g, &pl, why, 4);
}

hipError_t launch_stem_s2d_qi32(const Geom& g, const int8_t* x, const int8_t* w, const int32_t* T,
                                const int32_t* qrec, int32_t* y, hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  S2dPlan pl;
  if (!sd_plan(g, &pl, nullptr, 4)) return hipErrorInvalidConfiguration;
  const S2dArgs a = sd_args(g, pl, x, w, y, T, reinterpret_cast<const float*>(qrec), 1.0f);
  if (g.C == 3 && g.R == 7 && g.S == 7) {
    sd_go(i8_stem_s2d_kernel<4, false, 3, 7, 7, true>, a, pl, stream);
  } else {
    switch (pl.KB) {
      case 1: sd_go(i8_stem_s2d_kernel<1, false, 0, 0, 0, true>, a, pl, stream); break;
      case 2: sd_go(i8_stem_s2d_kernel<2, false, 0, 0, 0, true>, a, pl, stream); break;
      case 3: sd_go(i8_stem_s2d_kernel<3, false, 0, 0, 0, true>, a, pl, stream); break;
      default: sd_go(i8_stem_s2d_kernel<4, false, 0, 0, 0, true>, a, pl, stream); break;
    }
  }
  return hipGetLastError();
}

}  // namespace miq
