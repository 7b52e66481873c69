// int8 convolution for narrow feature maps (Wo <= 64) with small filters: row bands,
// filter-stationary MFMA (v_mfma_i32_16x16x64_i8), the band's input rows staged in LDS.
//
// Work decomposition.  A workgroup of 8 waves (two per SIMD) owns a band of BH consecutive
// output rows of one image and NT (1, 2, 4 or 8) consecutive 64-channel tiles of one group;
// WPT = 8 / NT waves work on each tile.  Output rows are cut into 16-pixel segments
// (segment column sc covers wo = 16*sc .. 16*sc + 15; the last one may be partly outside
// the image), numbered row-major over the band: s = t * SEGR + sc.  Wave wl of a tile
// computes segments wl, wl + WPT, wl + 2*WPT, ... (one per phase), advancing its input and
// output offsets incrementally.  The channel tile is the fastest index of the workgroup
// order, so the workgroups of one band run side by side and share its input rows in one
// XCD's L2.  A SIMD runs two waves so that one wave's LDS reads and epilogue overlap the
// other's MFMAs: one wave cannot overlap them with its own matrix instructions.  The host
// planner picks NT and BH by a cycle estimate: rounds of workgroups over the CUs x (phases
// x (MFMA + epilogue) + start-up + the loads of filter and rows).
//
// Filter-stationary.  Each wave keeps the whole 64-channel filter of the workgroup in
// registers: KB = R*S*Cg/64 K-blocks x 4 MFMA row blocks of 16 bytes per lane.  The only
// LDS traffic of the main loop is then the input fragments: 1 KB per K-block per segment,
// shared by the 64 output channels of the 4 MFMAs that consume it.
//
// Input rows.  The band's input rows (its "halo": (BH-1)*sh + (R-1)*dh + 1 rows) go to
// LDS as [row][chunk quad][16-column block][chunk in quad][column in block] x 16 bytes,
// halo column c holding input column c - pw (a chunk is 16 channels, a quad 4 chunks).
// One buffer_load_dwordx4 ... lds (global -> LDS without registers) fills one (row, quad,
// block): its 64 lanes read 16 pixels x 64 channel bytes, one contiguous kilobyte of NHWC
// input when the group has 64 channels.  The buffer range check turns every padding
// position into zeros (an out-of-image row or column gets an offset past num_records), so
// no lane is predicated.  The 16 lanes of an MFMA lane group
// read 16 consecutive columns of one chunk: their 16-byte slots are distinct modulo 16,
// so the read is free of bank conflicts for any column shift.
//
// Loads.  Every load of the workgroup (the band's input rows, epilogue parameters, filter)
// is issued at the start, spread over the 8 waves, with one buffer resource per tensor and
// a few scalar instructions per load: scalar work is shared by the waves of a SIMD and a
// long scalar loop delays everything behind it.  Kernel arguments are preloaded in one
// s_load batch.  The filter goes first (L2 after the first workgroup: it lands early),
// then the rows phase 0 reads, the epilogue parameters and the other rows.  Loads complete
// in order, so a wave waits (vmcnt) for the filter alone, a barrier publishes it, and every
// wave copies the whole filter into its registers while the rows are still arriving from
// HBM; a second wait and barrier publish phase 0's rows and the epilogue parameters, so
// phase 0 runs with the filter already in registers (measured against the rows first and
// a copy two K-blocks ahead of phase 0's MFMAs: C2 7.41 -> 7.28 us, C3 11.98 -> 11.25 us);
// after phase 0's MFMAs a third wait and barrier publish the other rows, and the phases
// run without synchronisation.
//
// Skew.  The two waves of a SIMD (w and w + 4) are offset by one epilogue: the leading
// wave runs MFMA(p) then epilogue(p), the trailing one epilogue(p - 1) then MFMA(p), so one
// wave's VALU work runs beside the other's matrix instructions.  The wait for the remaining
// rows after phase 0 realigns them (both then run epilogue 0, MFMA 1, ...); the trailing
// wave taking MFMA(p) first keeps them apart, but measured slower in graph replay
// (C2 7.27 -> 7.41 us).
//
// Epilogue.  Accumulators start at the bias; the output is convert, scale, clamp, round
// (the 1.5*2^23 addition, four results packed with two v_perm_b32 and an or) and one
// 16-byte store of 16 consecutive channels per lane, the arithmetic of the other int8
// kernels.  Every 16-byte store is followed by store_gap() on its data registers.

#include "qconv_device.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>

namespace miq {
namespace {

constexpr int kBandWaves = 8;  // two per SIMD: one wave's LDS reads and epilogue overlap the other's MFMAs
constexpr int kBandMaxKB = 9;  // filter registers per lane: 16 * KB
constexpr int kBandLds = 160 * 1024;

// LDS of one 64-channel tile's filter, in 16-byte slots: 4 * KB kilobytes, plus one for the
// block shifts of the contiguous (odd KB) layout
__host__ __device__ constexpr int band_tile_slots(int KB) { return 64 * (4 * KB + (KB & 1)); }

struct BandArgs {
  const int8_t* x;
  const int8_t* w;
  const int32_t* bias;
  const float* wscale;
  void* y;
  int H, W, C, K, Ho, Wo;
  int ph, pw, sh;
  int Cg, Kg, Kdim;
  int BH;             // output rows per band
  int bands_per_img;  // ceil(Ho / BH)
  int NT, WPT;        // 64-channel tiles per workgroup, waves per tile (8 / NT)
  int kt_per_group;   // workgroup channel tiles (NT * 64 channels) per group
  int nblocks;        // workgroups of the launch (gridDim would be one more kernarg round trip)
  int NQ, NPB;        // chunk quads (Cg / 64) and 16-column blocks per input row
  int SEGR;           // 16-pixel segment columns per output row
  // per phase a wave's segment advances WPT = dT * SEGR + dS segments: its input offset
  // by d_rb bytes and its output offset by d_out elements, plus c_rb / c_out when the
  // column wraps past the row's end
  int dS, d_rb, c_rb, d_out, c_out;
  int ni;             // input load instructions per workgroup = HR * NQ * NPB
  int ni0;            // those of the input rows phase 0 reads
  int filt_lds, ep_lds, halo_lds;  // LDS byte offsets
  float act_scale;
  int relu;
  // per K-block: LDS slot offset of its (filter row, chunk quad) << 8 | halo column shift
  // (filter column * dilation, < 256); the struct stays within 64 words, one s_load batch
  int tap[kBandMaxKB];
  int ntiles;         // workgroup channel tiles per band: groups * kt_per_group
  FastDivM fd_ntiles, fd_bpi, fd_ktpg, fd_rowi, fd_npb;
};

static_assert(sizeof(BandArgs) <= 256, "kernel arguments fit one s_load batch");

// MT: more than one 64-channel tile per workgroup (NT > 1); the single-tile
// instantiation keeps its tile arithmetic at compile time
template <int KB, int EPI, bool MT>
__global__ void __launch_bounds__(64 * kBandWaves, 1) i8_band_kernel(BandArgs a_in) {
  const BandArgs a = preload_args(a_in);
  // Channel order of the MFMA rows.  int8 outputs: row block j, row rho <-> channel
  // 16 * (rho / 4) + 4j + rho % 4, so a lane holds 16 consecutive channels (one 16-byte
  // store).  4-byte outputs: natural order (channel 16j + rho), so the 4 lanes of a pixel
  // store 64 contiguous bytes per instruction; 16-byte pieces 64 bytes apart, as the int8
  // order would give, ran the int32 output of C2 at 45.6 us against 7 us for int8.
  constexpr bool NAT = EPI != kEpiI8;
  const int NT = MT ? a.NT : 1;
  const int WPT = MT ? a.WPT : kBandWaves;
  extern __shared__ v4i smem[];
  v4i* filt = smem + a.filt_lds / 16;
  v4i* halo = smem + a.halo_lds / 16;
  v4i* ep = smem + a.ep_lds / 16;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row_l = lane & 15;
  const int grp_l = lane >> 4;

  const int lin = xcd_tile(blockIdx.x, a.nblocks);
  // channel tile fastest: the tiles of one band (which read the same input rows) get
  // neighbouring indices and so one XCD's L2
  const int band = fdiv(lin, a.fd_ntiles);
  const int ctile = lin - band * a.ntiles;
  const int n = fdiv(band, a.fd_bpi);
  const int bi = band - n * a.bands_per_img;
  const int gi = fdiv(ctile, a.fd_ktpg);
  const int k0 = (ctile - gi * a.kt_per_group) * NT * 64;  // first channel (in group gi)
  const int ho0 = bi * a.BH;
  // wave -> 64-channel tile tw of the workgroup, and its rank wl among the tile's waves
  const int tw = MT ? wave / WPT : 0;
  const int wl = wave - tw * WPT;
  const int row_instr = a.NQ * a.NPB;  // input load instructions per input row

  // Scalar work is shared by the waves of a SIMD (one instruction per wave per issue
  // turn), so the loads below use one buffer resource each and keep per-load work to a
  // few instructions.
  //
  // Issue order: the filter (L2 after the first workgroup), the input rows phase 0 reads,
  // the epilogue parameters, then the remaining rows.  A CU's vector memory path accepts
  // about 35 bytes per clock and loads complete in order, so what is issued first lands
  // first.
  //
  // ---- every input row of the band, in row order: instruction i = (row * NQ + quad) *
  // NPB + block goes to wave i % 8; its lane l reads column 16 * block + l % 16 - pw, chunk
  // 4 * quad + l / 16.  One resource covers the image (group gi's channels onward); the row
  // goes into soffset.  A column outside the image gets voffset 2^30 and a row outside it
  // soffset 2^30: either way past num_records (< 2^30), and their sum cannot wrap.
  const int hi0 = ho0 * a.sh - a.ph;
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(a.x + static_cast<size_t>(n) * a.H * a.W * a.C + static_cast<size_t>(gi) * a.Cg,
                a.H * a.W * a.C - gi * a.Cg);
  const int col_lane = row_l - a.pw;
  auto load_rows = [&](int i, int i_end) {
    int cnt = 0;
    for (; i < i_end; i += kBandWaves) {
      const int hr = fdiv(i, a.fd_rowi);
      const int rem = i - hr * row_instr;
      const int q = fdiv(rem, a.fd_npb);
      const int pb = rem - q * a.NPB;
      const int hi = hi0 + hr;
      const unsigned soff =
          static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) ? static_cast<unsigned>(hi * a.W * a.C + 64 * q) : 0x40000000u;
      const int col = col_lane + 16 * pb;
      const unsigned voff =
          static_cast<unsigned>(col) < static_cast<unsigned>(a.W) ? static_cast<unsigned>(col * a.C + 16 * grp_l) : 0x40000000u;
      load_lds16(rx, halo + i * 64, voff, soff);
      ++cnt;
    }
    return cnt;
  };
  // ---- filter -> LDS, instruction f to wave f % 8.  Even KB: fragment order; fragment
  // f = 4KB*t + 4b + j (64-channel tile t, K-block b, MFMA row block j) is one
  // instruction, whose lane (row_l, grp_l) holds channel
  // k0 + 64t + 16*(row_l/4) + 4j + row_l%4, bytes [16*(4b + grp_l), +16) of that channel's
  // KRSC row; channels at or beyond Kg lie past num_records (zeros).
  //
  // Odd KB: the tile's 64 KRSC rows (64 * Kdim = 4 * KB kilobytes) are one contiguous
  // range, loaded as it lies, 1 KB per instruction (the fastest global -> LDS form).  A
  // block of 16 channels is KB instructions; blocks 2 and 3 land 2 slots (32 bytes)
  // further on.  A ds_read_b128 serves 16 lanes per cycle: one half-wave's lane quads of
  // equal quad-index parity.  A fragment read then gives each cycle the slots
  // 4 * (KB * a mod 4) + grp_l + 2 * (m / 2) + const modulo 16 for channels 16m + 4j + a,
  // all distinct: no bank conflicts.
  {
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + static_cast<size_t>(gi) * a.Kg * a.Kdim, a.Kg * a.Kdim);
    if constexpr (KB & 1) {
      for (int f = wave; f < NT * 4 * KB; f += kBandWaves) {
        const int t = MT ? f / (4 * KB) : 0;
        const int u = f - t * (4 * KB);
        load_lds16(rw, filt + t * band_tile_slots(KB) + 64 * u + 2 * ((u / KB) >> 1), 16u * lane,
                   static_cast<unsigned>((k0 + 64 * t) * a.Kdim + 1024 * u));
      }
    } else {
      const int rl = NAT ? row_l : 16 * (row_l >> 2) + (row_l & 3);
      const unsigned lane_row = static_cast<unsigned>(rl * a.Kdim + 16 * grp_l);
      for (int f = wave; f < NT * 4 * KB; f += kBandWaves) {
        const int t = MT ? f / (4 * KB) : 0;
        const int ff = f - t * (4 * KB);
        load_lds16(rw, filt + f * 64, lane_row,
                   static_cast<unsigned>((k0 + 64 * t + (NAT ? 16 : 4) * (ff & 3)) * a.Kdim + 64 * (ff >> 2)));
      }
    }
  }
  const int row0_loads = load_rows(wave, a.ni0);
  // ---- bias and per-channel scales of tile t's 64 channels (wave t), 2 KB of LDS each ----
  if (EPI != kEpiAcc32 && wave < NT) {
    const int kt = k0 + 64 * wave;
    const int valid = max(0, a.Kg - kt) * 4;
    const size_t off = static_cast<size_t>(gi) * a.Kg + min(kt, a.Kg);
    load_lds16(make_rsrc(a.bias ? a.bias + off : nullptr, a.bias ? valid : 0), ep + 128 * wave, 16u * lane, 0);
    load_lds16(make_rsrc(a.wscale + off, valid), ep + 128 * wave + 64, 16u * lane, 0);
  }
  // ---- the remaining input rows (instructions ni0 .. ni - 1, wave i % 8) ----
  const int first_rest = a.ni0 + ((wave - a.ni0) % kBandWaves + kBandWaves) % kBandWaves;
  const int rest_loads = load_rows(first_rest, a.ni);
  // phase 0's rows, the epilogue parameters and the filter (everything but the remaining
  // rows) complete; the barrier publishes every wave's part
  const int ep_loads = (EPI != kEpiAcc32 && wave < NT) ? 2 : 0;
  wait_vmcnt(row0_loads + ep_loads + rest_loads);  // the filter (issued first) has landed
  barrier_only();

  // The filter stays in registers: A[b][j] is K-block b, MFMA row block j, copied from LDS
  // while the input rows are still arriving from HBM.
  v4i A[KB][4];
  // lane (row_l, grp_l) of fragment (b, j), odd KB: channel n = 16 * (row_l / 4) + 4j +
  // row_l % 4 of the tile, 16-byte unit 4 * KB * n + 4b + grp_l, plus its block's shift
  // (natural order: channel n = 16j + row_l, unit 4 * KB * n + 4b + grp_l + 2 * (j / 2))
  const v4i* ft = NAT ? filt + tw * band_tile_slots(KB) + 4 * KB * row_l + grp_l
                      : filt + tw * band_tile_slots(KB) + 4 * KB * (16 * (row_l >> 2) + (row_l & 3)) + grp_l +
                            2 * (row_l >> 3);
  auto read_A = [&](int b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr ((KB & 1) && NAT)
        A[b][j] = ft[64 * KB * j + 2 * (j >> 1) + 4 * b];
      else if constexpr (KB & 1)
        A[b][j] = ft[16 * KB * j + 4 * b];
      else
        A[b][j] = filt[(tw * 4 * KB + b * 4 + j) * 64 + lane];
    }
  };
#pragma unroll
  for (int b = 0; b < KB; ++b) read_A(b);
  wait_vmcnt(rest_loads);  // phase 0's rows and the epilogue parameters
  barrier_only();
  // epilogue parameters of this lane's 16 channels (zero past Kg): kc0 + 4j + r, or in
  // natural order kt0 + 16j + 4 grp_l + r
  const int kt0 = k0 + 64 * tw;
  const int kc0 = kt0 + 16 * grp_l;
  const bool ch_ok = kc0 < a.Kg;  // Kg % 16 == 0: a lane's 16 channels all exist or none does
  const int nj_ok = min(4, (a.Kg - kt0) >> 4);  // natural order: row blocks inside the group
  v4i bias_v[4];
  v4f mult_v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bias_v[j] = v4i{0, 0, 0, 0};
    mult_v[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (EPI != kEpiAcc32) {
      const int ev = NAT ? 4 * j + grp_l : 4 * grp_l + j;
      bias_v[j] = ep[128 * tw + ev];
      const v4i ws = ep[128 * tw + 64 + ev];
#pragma unroll
      for (int r = 0; r < 4; ++r) mult_v[j][r] = requant_multiplier(a.act_scale, __int_as_float(ws[r]));
    }
  }

  // Phase p of wave wl works on segment s = wl + p * WPT of the band's band_rows * SEGR
  // (row t = s / SEGR, segment column sc = s % SEGR: output columns 16 * sc + row_l).
  // LDS byte address of this lane's fragment of K-block b in segment (0, 0): column
  // x = row_l + shift lies in block x / 16 at position x % 16, i.e. slot
  // 64 * (x / 16) + x % 16 = x + 48 * (x / 16); plus its chunk and the K-block's row and
  // quad.  Segment (t, sc) adds the uniform t * row_bytes + sc * 1024.
  const unsigned halo_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(halo) & 0xffffffffu);
  unsigned baddr[KB];
#pragma unroll
  for (int b = 0; b < KB; ++b) {
    const int x = row_l + (a.tap[b] & 0xff);
    baddr[b] = halo_addr + 16u * static_cast<unsigned>((a.tap[b] >> 8) + 16 * grp_l + x + 48 * (x >> 4));
  }
  const unsigned row_bytes = 16u * static_cast<unsigned>(a.sh * row_instr * 64);  // per output row
  const float lo = a.relu ? 0.0f : -128.0f;

  // Output through a buffer resource over the band's rows (of image n, group gi): the lane
  // part of the offset is fixed, the segment part goes into soffset.  A lane whose pixel or
  // channels do not exist gets 2^30 more and its store is dropped.
  constexpr int kOutBytes = EPI == kEpiI8 ? 1 : 4;
  const int band_rows = min(a.BH, a.Ho - ho0);
  const size_t out0 = (static_cast<size_t>(n) * a.Ho + ho0) * a.Wo * a.K + static_cast<size_t>(gi) * a.Kg;
  const __amdgpu_buffer_rsrc_t ry =
      make_rsrc(static_cast<char*>(a.y) + out0 * kOutBytes, band_rows * a.Wo * a.K * kOutBytes);
  const unsigned lane_out = NAT ? static_cast<unsigned>((row_l * a.K + kt0 + 4 * grp_l) * kOutBytes)
                               : static_cast<unsigned>((row_l * a.K + kc0) * kOutBytes) + (ch_ok ? 0u : 0x40000000u);
  const int nseg = band_rows * a.SEGR;
  // The segment (row t, column seg_c) of the current phase, walked forward by WPT segments
  // per phase: its input offset seg_in (t * row_bytes + 1024 * seg_c), output soffset
  // seg_out ((t * Wo + 16 * seg_c) * K elements) and this lane's output offset (2^30 more
  // for a pixel past the row's end: only the last column can hold one).
  int seg_t = 0, seg_c = wl;  // wl < 8: a few subtractions
  while (seg_c >= a.SEGR) {
    seg_c -= a.SEGR;
    ++seg_t;
  }
  unsigned seg_in = static_cast<unsigned>(seg_t) * row_bytes + 1024u * static_cast<unsigned>(seg_c);
  int seg_out = (seg_t * a.Wo + 16 * seg_c) * a.K;
  const unsigned lane_last = lane_out + (16 * (a.SEGR - 1) + row_l < a.Wo ? 0u : 0x40000000u);
  auto seg_rb = [&]() { return seg_in; };
  auto seg_soff = [&]() { return static_cast<unsigned>(seg_out * kOutBytes); };
  auto seg_lane = [&]() { return seg_c == a.SEGR - 1 ? lane_last : lane_out; };
  auto seg_next = [&]() {
    seg_c += a.dS;
    seg_in += static_cast<unsigned>(a.d_rb);
    seg_out += a.d_out;
    if (seg_c >= a.SEGR) {
      seg_c -= a.SEGR;
      seg_in += static_cast<unsigned>(a.c_rb);
      seg_out += a.c_out;
    }
  };
  auto emit = [&](const v4i (&acc)[4], unsigned soff, unsigned lane_out_q) {
    if constexpr (EPI == kEpiI8) {
      const v4i pk = a.relu ? pack_u8_relu(acc, mult_v) : pack_i8(acc, mult_v, lo);
      __builtin_amdgcn_raw_buffer_store_b128(pk, ry, lane_out_q, soff, kStoreAux);
      store_gap(pk);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j >= nj_ok) break;  // natural order: channels 16j .. past the group
        v4i v = acc[j];
        if constexpr (EPI == kEpiF32) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float f = static_cast<float>(acc[j][r]) * mult_v[j][r];
            if (a.relu) f = (f > 0.0f) ? f : 0.0f;  // NaN and -0 -> +0
            v[r] = __float_as_int(f);
          }
        }
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, lane_out_q + 64 * j, soff, kStoreAux);
        store_gap(v);
      }
    }
  };
  auto mfma_phase = [&](unsigned rb, v4i (&acc)[4]) {
    // input fragments are read RS K-blocks ahead: each read goes out right after the
    // MFMAs that free its register
    constexpr int RS = KB < 4 ? KB : 4;
    v4i B[RS];
#pragma unroll
    for (int r = 0; r < RS; ++r) B[r] = lds_read16(baddr[r] + rb);
#pragma unroll
    for (int b = 0; b < KB; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][j], B[b % RS], b == 0 ? bias_v[j] : acc[j], 0, 0, 0);
      }
      if (b + RS < KB) B[b % RS] = lds_read16(baddr[b + RS] + rb);
      __builtin_amdgcn_sched_barrier(0);  // keeps each read RS K-blocks ahead of its use
    }
  };
  // The wait for the remaining rows comes after the phase-0 MFMAs and before the first
  // store (exact: no store is pending yet), and after its barrier nothing synchronises
  // any more.
  auto wait_rest = [&]() {
    wait_vmcnt(0);
    barrier_only();
  };
  // The two waves of a SIMD (waves w and w + 4) are skewed by one epilogue: the "leading"
  // wave w < 4 runs MFMA(p) then the epilogue of p; the trailing one runs the epilogue of
  // p - 1 then MFMA(p), so one wave's VALU work runs beside the other's matrix instructions.
  const int nph = wl < nseg ? (nseg - wl + WPT - 1) / WPT : 0;
  v4i acc[4];
  if (wave < kBandWaves / 2) {
    for (int p = 0; p < nph; ++p) {
      mfma_phase(seg_rb(), acc);
      if (p == 0) wait_rest();
      emit(acc, seg_soff(), seg_lane());
      seg_next();
    }
    if (nph == 0) wait_rest();
  } else {
    unsigned soff_prev = 0, lane_prev = 0;  // the previous phase's output offsets
    for (int p = 0; p < nph; ++p) {
      v4i prev[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) prev[j] = acc[j];
      if (p == 1) wait_rest();
      if (p > 0) emit(prev, soff_prev, lane_prev);
      mfma_phase(seg_rb(), acc);
      soff_prev = seg_soff();
      lane_prev = seg_lane();
      seg_next();
    }
    if (nph <= 1) wait_rest();
    if (nph > 0) emit(acc, soff_prev, lane_prev);
  }
}
struct BandPlan {
  int KB, NQ, NPB, SEGR, NT, WPT, BH, bands_per_img, kt_per_group, HR, ni, ni0;
  int filt_lds, ep_lds, halo_lds;
  size_t lds_bytes;
};

int band_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

bool band_plan(const Geom& g, Epi epi, BandPlan* p, std::string* why) {
  auto no = [&](const char* m) { if (why) *why = m; return false; };
  if (g.Cg % 64 != 0 || g.Cg == 0) return no("band kernel needs (c/groups) % 64 == 0");
  if (g.Kg <= 0 || g.Kg % 16 != 0) return no("band kernel needs (k/groups) % 16 == 0");
  if (g.sw != 1) return no("band kernel needs stride_w == 1");
  if (g.sh < 1 || g.dh < 1 || g.dw < 1 || g.ph < 0 || g.pw < 0) return no("band kernel needs positive stride/dilation");
  if (g.Wo > 64) return no("band kernel needs output width <= 64");
  if (g.R < 1 || g.S < 1) return no("band kernel needs a non-empty filter");
  const long long kb = static_cast<long long>(g.R) * g.S * (g.Cg / 64);
  if (kb > kBandMaxKB) return no("band kernel filter does not fit in registers (R*S*c/groups > 576)");
  if (static_cast<long long>(g.H) * g.W * g.C >= (1LL << 30)) return no("band kernel needs images below 2^30 bytes");
  if (static_cast<long long>(g.Kg) * g.R * g.S * g.Cg >= (1LL << 30)) return no("band kernel needs group filters below 2^30 bytes");
  if (static_cast<long long>(g.Ho) * g.Wo * g.K * 4 >= (1LL << 30)) return no("band kernel needs images below 2^30 output bytes");
  const long long hcols = static_cast<long long>(g.Wo) + static_cast<long long>(g.S - 1) * g.dw;
  if (hcols > 128) return no("band kernel needs output width + dilated filter width <= 128");
  p->KB = static_cast<int>(kb);
  p->NQ = g.Cg / 64;
  p->NPB = static_cast<int>((hcols + 15) / 16);
  p->SEGR = (g.Wo + 15) / 16;
  const int kt64 = (g.Kg + 63) / 64;  // 64-channel tiles per group
  const int cus = band_cu_count();
  // Cost in cycles of one round of workgroups (one per CU): the busiest SIMD runs two
  // waves whose matrix instructions and epilogue VALU work do not overlap (measured), so
  // a phase costs KB * 4 MFMAs of 16 cycles plus about 450 cycles of epilogue, twice;
  // loading the filter and the input rows costs about a cycle per 25 bytes plus a fixed
  // 2400 (launch, first loads, barriers).
  bool found = false;
  double best = 0.0;
  for (int nt = 1; nt <= kBandWaves; nt *= 2) {
    if (kt64 % nt != 0) continue;
    const int wpt = kBandWaves / nt;
    const size_t filt_bytes = static_cast<size_t>(nt) * band_tile_slots(p->KB) * 16;
    for (int bh = 1; bh <= g.Ho; ++bh) {
      const long long hr = static_cast<long long>(bh - 1) * g.sh + static_cast<long long>(g.R - 1) * g.dh + 1;
      const long long ni = hr * p->NQ * p->NPB;
      if (ni > kBandWaves * 15) break;  // at most 15 input loads per wave (exact vmcnt waits)
      const size_t lds = filt_bytes + static_cast<size_t>(nt) * 2048 + static_cast<size_t>(ni + 1) * 1024;
      if (lds > static_cast<size_t>(kBandLds)) break;
      const long long bands = (g.Ho + bh - 1) / bh;
      const long long wgs = static_cast<long long>(g.N) * bands * g.G * (kt64 / nt);
      const long long rounds = (wgs + cus - 1) / cus;
      const long long nph = (static_cast<long long>(bh) * p->SEGR + wpt - 1) / wpt;
      const double phase = p->KB * 64.0 + 450.0;
      const double load = 2400.0 + static_cast<double>(filt_bytes + ni * 1024) / 25.0;
      const double cost = static_cast<double>(rounds) * (2.0 * static_cast<double>(nph) * phase + load);
      if (!found || cost < best - 1e-9) {
        found = true;
        best = cost;
        p->NT = nt;
        p->WPT = wpt;
        p->kt_per_group = kt64 / nt;
        p->BH = bh;
        p->bands_per_img = static_cast<int>(bands);
        p->HR = static_cast<int>(hr);
        p->ni = static_cast<int>(ni);
        // input rows the first phase of every wave reads: segments 0 .. WPT-1
        const long long rows0 = std::min<long long>(hr, static_cast<long long>((wpt - 1) / p->SEGR) * g.sh +
                                                            static_cast<long long>(g.R - 1) * g.dh + 1);
        p->ni0 = static_cast<int>(rows0 * p->NQ * p->NPB);
        p->filt_lds = 0;
        p->ep_lds = static_cast<int>(filt_bytes);
        p->halo_lds = static_cast<int>(filt_bytes + static_cast<size_t>(nt) * 2048);
        p->lds_bytes = lds;
      }
    }
  }
  if (!found) return no("band kernel input rows do not fit in LDS");
  const long long blocks = static_cast<long long>(g.N) * p->bands_per_img * g.G * p->kt_per_group;
  if (blocks > 0x7fffffffLL) return no("grid too large");
  return true;
}

template <int KB>
void band_launch_kb(const BandArgs& a, const BandPlan& pl, Epi epi, unsigned nblocks, hipStream_t stream) {
  const dim3 grid(nblocks);
  switch (epi) {
    case kEpiI8: {
      auto kern = pl.NT > 1 ? i8_band_kernel<KB, kEpiI8, true> : i8_band_kernel<KB, kEpiI8, false>;
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(pl.lds_bytes));
      hipLaunchKernelGGL(kern, grid, dim3(64 * kBandWaves), pl.lds_bytes, stream, a);
      break;
    }
    case kEpiAcc32: {
      auto kern = pl.NT > 1 ? i8_band_kernel<KB, kEpiAcc32, true> : i8_band_kernel<KB, kEpiAcc32, false>;
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(pl.lds_bytes));
      hipLaunchKernelGGL(kern, grid, dim3(64 * kBandWaves), pl.lds_bytes, stream, a);
      break;
    }
    default: {
      auto kern = pl.NT > 1 ? i8_band_kernel<KB, kEpiF32, true> : i8_band_kernel<KB, kEpiF32, false>;
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(pl.lds_bytes));
      hipLaunchKernelGGL(kern, grid, dim3(64 * kBandWaves), pl.lds_bytes, stream, a);
      break;
    }
  }
}

template <int KB>
void band_dispatch(int kb, const BandArgs& a, const BandPlan& pl, Epi epi, unsigned nblocks, hipStream_t stream) {
  if constexpr (KB >= 1) {
    if (kb == KB) {
      band_launch_kb<KB>(a, pl, epi, nblocks, stream);
    } else {
      band_dispatch<KB - 1>(kb, a, pl, epi, nblocks, stream);
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool band_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                   std::string* why) {
  const bool params_ok = epi == kEpiAcc32 || ((rq.bias == nullptr || aligned16(rq.bias)) && aligned16(rq.wscale));
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || !params_ok) {
    if (why) *why = "band kernel needs 16-byte aligned tensors, bias and scales";
    return false;
  }
  BandPlan pl;
  return band_plan(g, epi, &pl, why);
}

hipError_t launch_i8_band(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  BandPlan pl;
  if (!band_plan(g, epi, &pl, nullptr)) return hipErrorInvalidConfiguration;
  BandArgs a;
  a.x = x; a.w = w; a.bias = rq.bias; a.wscale = rq.wscale; a.y = y;
  a.H = g.H; a.W = g.W; a.C = g.C; a.K = g.K; a.Ho = g.Ho; a.Wo = g.Wo;
  a.ph = g.ph; a.pw = g.pw; a.sh = g.sh;
  a.Cg = g.Cg; a.Kg = g.Kg; a.Kdim = g.R * g.S * g.Cg;
  a.BH = pl.BH; a.bands_per_img = pl.bands_per_img; a.NT = pl.NT; a.WPT = pl.WPT;
  a.kt_per_group = pl.kt_per_group; a.NQ = pl.NQ; a.NPB = pl.NPB; a.SEGR = pl.SEGR;
  a.ni = pl.ni; a.ni0 = pl.ni0;
  a.filt_lds = pl.filt_lds; a.ep_lds = pl.ep_lds; a.halo_lds = pl.halo_lds;
  a.act_scale = rq.act_scale; a.relu = rq.relu;
  // K-block b = chunks 4b .. 4b+3 of the flattened (tap, 16-channel chunk) order, all of
  // one tap because Cg16 % 4 == 0.
  const int cg16 = g.Cg / 16;
  for (int b = 0; b < kBandMaxKB; ++b) {
    if (b < pl.KB) {
      const int q0 = 4 * b;
      const int tap = q0 / cg16;
      const int cb = q0 % cg16;
      const int r = tap / g.S;
      const int s = tap % g.S;
      a.tap[b] = ((r * g.dh * pl.NQ + cb / 4) * pl.NPB * 64) << 8 | (s * g.dw);
    } else {
      a.tap[b] = 0;
    }
  }
  a.ntiles = g.G * pl.kt_per_group;
  a.fd_ntiles = fastdiv_m(a.ntiles);
  a.fd_bpi = fastdiv_m(pl.bands_per_img);
  a.fd_ktpg = fastdiv_m(pl.kt_per_group);
  a.fd_rowi = fastdiv_m(pl.NQ * pl.NPB);
  a.fd_npb = fastdiv_m(pl.NPB);
  {
    const int dT = pl.WPT / pl.SEGR;
    const int row_bytes = g.sh * pl.NQ * pl.NPB * 1024;  // LDS bytes of sh input rows
    a.dS = pl.WPT % pl.SEGR;
    a.d_rb = dT * row_bytes + 1024 * a.dS;
    a.c_rb = row_bytes - 1024 * pl.SEGR;
    a.d_out = (dT * g.Wo + 16 * a.dS) * g.K;
    a.c_out = (g.Wo - 16 * pl.SEGR) * g.K;
  }
  const long long nblocks = static_cast<long long>(g.N) * pl.bands_per_img * g.G * pl.kt_per_group;
  a.nblocks = static_cast<int>(nblocks);
  band_dispatch<kBandMaxKB>(pl.KB, a, pl, epi, static_cast<unsigned>(nblocks), stream);
  return hipGetLastError();
}

}  // namespace miq
