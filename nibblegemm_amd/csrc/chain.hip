// Persistent decode chain: a list of strip-major decode GEMVs ("stages"), each
// of which may have to wait for an earlier one, run by ONE launch.
//
// No counterpart in the reference.  Its batch-1 decode step is one launch per
// projection (bench/bench_model.py:70-86), and it names the fix for the
// launch-bound small projections as structural: fewer launches
// (docs/OPTIMIZATION_LOG.md:159-163).  On MI355X a graph-replayed launch of
// the strip kernel costs ~3.5 us beyond its weight stream at K = 4096 (launch,
// first HBM round trip, reduction, end-of-kernel release), so the 8B step's
// 128 launches spend about half of its time there.  This kernel keeps the
// weight stream going across projection boundaries instead.
//
// Workgroups are persistent: one per CU, 8 compute waves + 1 staging wave.
// The host assigns every workgroup an ordered list of rounds; a round is one
// strip of a stage for each "team" of the workgroup's compute waves (a team is
// the strip kernel's workgroup for that strip width: 4 waves for 64-column
// strips, so two strips per round, 8 waves for 16 and 32 columns).  Each
// wave of a team handles the same quant groups, in the same order, with the
// same MFMA sequence, and the staging wave sums the waves' partials in the
// same order as the strip kernel (gemv.hip), so every output has the bits of
// nibble_gemv_w4a16_strip_major on the same operands.
//
// Weight ring (compute waves).  Each compute wave owns kRing 1 KiB LDS slots
// and keeps exactly kRing direct-to-LDS buffer loads in flight: a wave load of
// a strip-major strip is 1 KiB contiguous (lane l's 16 bytes at byte 16 l),
// so the wave consumes slot i (s_waitcnt vmcnt(kRing - 1): the oldest load
// has landed), reads its 16 bytes into registers, and refills the slot with
// the next load of its sequence -- which runs on into the wave's next rounds,
// whatever their stage.  The weights do not depend on the activations, so
// they stream while the wave waits for the round's activations.  The compute
// waves issue no other vector-memory instruction, so the wait count is exact.
//
// Staging wave.  Everything that depends on another workgroup goes through
// it, so that its waits never hold back the compute waves' weight loads (a
// vector-memory wait waits for every older load of the wave):
//   * before round r: if the stage waits for an earlier stage, spin on that
//     stage's counter (round items finished) until it is complete; copy the
//     activation rows (and a bias slice) into LDS with agent-coherent LDS-DMA
//     loads (sc1: the producer's stores came from other XCDs), and the
//     strips' scales -- ahead of time, during round r - 1, where nothing has to
//     be waited for;
//   * after round r: sum the compute waves' partials from LDS, apply the
//     epilogue, store Y with agent-coherent stores, wait for them, and bump
//     the stage's counter.
// Every wait is bounded: past kSpinCap polls (or when another workgroup has
// already given up) the wave raises the chain's error flag, the workgroup
// stops after the current barrier, and nibble_chain_check reports it.  Rounds
// are assigned in stage order on every workgroup and the grid is at most one
// workgroup per CU (host-checked occupancy), so every stage a workgroup waits
// for is held by running workgroups that wait only for earlier stages.
//
// The last workgroup to finish resets the stage counters, so a chain can be
// replayed (eagerly or from a HIP graph) with no host work between runs.
// Ordering of the stores before the counter update relies on the gfx950
// behaviour described in nibble_decode.h ("HARDWARE ASSUMPTION").
#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "nibble_common.h"
#include "nibble_decode.h"
#include "nibble_epilogue.h"
#include "stream_matmul.h"

namespace nibble {
namespace {

constexpr int kComputeWaves = 8;
constexpr int kStagerWave = kComputeWaves;
constexpr int kChainThreads = (kComputeWaves + 1) * 64;
constexpr int kRing = 10;                 // 1 KiB weight slots per compute wave
constexpr uint32_t kSlotBytes = 1024;
constexpr uint32_t kRingBytes = kComputeWaves * kRing * kSlotBytes;
constexpr uint32_t kBiasBytes = 256;      // two strips of at most 64 fp16 biases
constexpr uint32_t kSpinCap = 1u << 18;   // polls of a counter before a wait gives up
constexpr int kPolicyNt = 2;              // buffer-load cache policy: non-temporal
constexpr int kPolicySc1 = 16;            // agent-coherent (misses a stale L2 line)
constexpr size_t kLdsMax = 160 * 1024;

constexpr int kWaitRingOldest = waitcnt_vm(kRing - 1);

// One stage as the kernel reads it (built and checked on the host).
struct ChainStage {
  const _Float16* X;     // [M, K]
  const uint32_t* Wt;    // words: strip s's packed row r at s * w_col + r * w_row
  const _Float16* St;    // scales: strip s's group g at s * s_col + g * s_row
  _Float16* Y;           // [M, N] (SwiGLU: [M, N / 2])
  const _Float16* bias;  // [N] for the bias epilogue
  uint32_t K, N;
  uint32_t sw;           // strip columns: 16, 32 or 64
  uint32_t groups;       // K / GROUP
  uint32_t w_strip, s_strip;  // bytes of one strip's words / scales
  uint32_t wbytes, sbytes;    // bytes of Wt / St
  uint32_t xbytes;            // M * K * 2
  uint32_t epilogue;
  int32_t after;              // stage that must be complete before this one reads, or -1
  uint32_t after_items;       // round items of that stage
  uint32_t signal;            // count this stage's finished round items
  // Strides of the weight layout: strip-major (w_col = w_strip, w_row =
  // 4 sw, s_col = s_strip, s_row = 2 sw) or packed (4 sw, 4 N, 2 sw, 2 N).
  uint32_t w_col, w_row, s_col, s_row;
  uint32_t pad;
};
static_assert(sizeof(ChainStage) == 112, "descriptor layout");

struct ChainArgs {
  const ChainStage* stages;
  const int4* rounds;       // {stage, strip of team 0, strip of team 1 (or -1), 0}
  const int* round_begin;   // [grid + 1]: workgroup w runs rounds [round_begin[w], round_begin[w + 1])
  uint32_t* counters;       // [n_stages] finished round items
  uint32_t* done;           // workgroups finished
  uint32_t* error;          // non-zero once a wait gave up (sticky until checked)
  // [n_stages + 1] or null: per stage the latest time one of its rounds was
  // emitted (atomic max), then the earliest start of a workgroup (atomic min);
  // s_memrealtime ticks (100 MHz).
  unsigned long long* stamps;
  int M;
  int n_stages;
  uint32_t xbuf_halves;     // one activation buffer: MT * max K fp16
  uint32_t sbuf_bytes;      // one scale buffer
};

__device__ __forceinline__ uint32_t load_coherent_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The plan (descriptors and round lists) is read-only for a launch: read
// through the constant address space, so wave-uniform reads become scalar
// loads (s_load), which the compute waves' vector-memory wait counts never
// see.
#if defined(__HIP_DEVICE_COMPILE__)
template <typename T>
using const_ptr = const __attribute__((address_space(4))) T*;
#else
template <typename T>
using const_ptr = const T*;  // the host pass only parses the kernels
#endif
template <typename T>
__device__ __forceinline__ const_ptr<T> as_const(const T* p) {
  return (const_ptr<T>)(p);
}

__device__ __forceinline__ f4_t mfma16c(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The waves and phases of a strip width (the strip kernel's plan for
// strip-major weights: 4 waves for 64-column strips, 8 otherwise).
__host__ __device__ constexpr int chain_waves(int sw) { return sw == 64 ? 4 : 8; }

// One round of one compute wave: the strip kernel's per-wave loop (prep,
// decode, MFMAs, per-group scaling) over the wave's quant groups, with the
// weights taken from the ring, then its partials written to `red`.
template <int MT, int GROUP, int SW, typename Take>
__device__ __forceinline__ void chain_round(const ChainStage& st, int strip, int wave,
                                            uint32_t lane, const _Float16* xb,
                                            const _Float16* sb, float* red, Take&& take) {
  constexpr int WAVES = chain_waves(SW);
  constexpr int LPR = SW / 4;
  constexpr int RPL = 64 / LPR;
  constexpr int P = RPL / 4;
  constexpr int KPL = 8 * RPL;
  constexpr int CPG = GROUP / KPL;
  constexpr int RPT = 16 / P;
  constexpr int TILES = (MT + RPT - 1) / RPT;
  constexpr int LANE_ROWS = MT < 4 ? MT : 4;
  static_assert(CPG >= 1 && GROUP % KPL == 0, "a wave load must not straddle quant groups");
  const int team = wave / WAVES, wt = wave % WAVES;
  const uint32_t K = st.K, groups = st.groups;
  const uint32_t g0 = wt * groups / WAVES, g1 = (wt + 1) * groups / WAVES;
  const uint32_t c = lane % LPR;
  const uint32_t mq = lane & 15u, kb = lane >> 4;
  const uint32_t ph = mq / RPT, mm = mq % RPT;
  const uint32_t kx_lane = (kb * P + ph) * 8u;
  const _Float16* s_team = sb + team * groups * SW;
  (void)strip;

  f4_t tot[TILES][4];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) tot[t][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const DecodeConsts dk = decode_consts();
  const h8_t xscale = biased_x_scale();
  const h8_t bcorr = biased_correction();

  for (uint32_t g = g0; g < g1; ++g) {
    h8_t x[TILES][CPG];
    f4_t corr[TILES];
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      // A rows past the block read row MT - 1: their MFMA rows are never kept.
      const uint32_t row = t * RPT + mm < MT ? t * RPT + mm : MT - 1;
      f4_t cr = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int cc = 0; cc < CPG; ++cc) {
        x[t][cc] = *reinterpret_cast<const h8_t*>(&xb[row * K + g * GROUP + cc * KPL + kx_lane]) *
                   xscale;
        cr = mfma16c(x[t][cc], bcorr, cr);
      }
      corr[t] = cr;
    }
    const h4_t sc = *reinterpret_cast<const h4_t*>(&s_team[g * SW + 4 * c]);
    f4_t acc[TILES][4];
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][j] = corr[t];
#pragma unroll
    for (int cc = 0; cc < CPG; ++cc) {
      const u4_t w = take();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h8_t b = decode8_biased(w[j], dk);
#pragma unroll
        for (int t = 0; t < TILES; ++t) acc[t][j] = mfma16c(x[t][cc], b, acc[t][j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sj = static_cast<float>(sc[j]);
#pragma unroll
      for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int i = 0; i < LANE_ROWS; ++i)
          tot[t][j][i] = __builtin_fmaf(sj, acc[t][j][i], tot[t][j][i]);
    }
  }

  // Lane (n = lane % 16, row block lane / 16) keeps the C entries of its own
  // phase: red[wave][phase][row][column].
  const int nslot = lane & 15;
  const int my_phase = nslot / LPR;
  const int ccol = 4 * (nslot % LPR);
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int i = 0; i < LANE_ROWS; ++i) {
      const int mp = 4 * (lane >> 4) + i;
      const int m = t * RPT + mp % RPT;
      if (mp / RPT == my_phase && m < MT) {
#pragma unroll
        for (int j = 0; j < 4; ++j) red[((wave * P + my_phase) * MT + m) * SW + ccol + j] = tot[t][j][i];
      }
    }
}

// The staging wave's output stage for a round of strip width SW: partials
// summed in (wave, phase) order per team -- the strip kernel's order --
// through the stage's epilogue, stored agent-coherently.
template <int MT, int SW>
__device__ __forceinline__ void chain_emit(const ChainStage& st, int4 rd, int M, uint32_t lane,
                                           const float* red, const _Float16* bb) {
  constexpr int WAVES = chain_waves(SW);
  constexpr int P = (64 / (SW / 4)) / 4;
  constexpr int TEAMS = kComputeWaves / WAVES;
  constexpr int QUADS = SW / 4;
  constexpr int E = WAVES * P;
  auto total = [&](int team, int r, int qq) {
    f4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int w = team * WAVES + e / P;
      const f4_t v =
          *reinterpret_cast<const f4_t*>(&red[((w * P + e % P) * MT + r) * SW + 4 * qq]);
      sum[0] += v[0];
      sum[1] += v[1];
      sum[2] += v[2];
      sum[3] += v[3];
    }
    return sum;
  };
  auto store = [](_Float16* dst, h4_t y) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(dst), __builtin_bit_cast(uint64_t, y),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if constexpr (SW >= 2 * kSwigluBlock) {
    if (st.epilogue == kEpilogueSwiglu) {
      constexpr int OUT = QUADS / 2;  // output quads per strip
      const uint32_t nout = st.N / 2;
      for (int e = lane; e < MT * TEAMS * OUT; e += 64) {
        const int r = e / (TEAMS * OUT), team = (e / OUT) % TEAMS, o = e % OUT;
        const int strip = team == 0 ? rd.y : rd.z;
        if (r >= M || strip < 0) continue;
        const int gq = 8 * (o / 4) + o % 4;
        const f4_t g = total(team, r, gq), u = total(team, r, gq + 4);
        const h4_t y = {(_Float16)silu_mul(g[0], u[0]), (_Float16)silu_mul(g[1], u[1]),
                        (_Float16)silu_mul(g[2], u[2]), (_Float16)silu_mul(g[3], u[3])};
        store(st.Y + static_cast<size_t>(r) * nout + strip * (SW / 2) + 4 * o, y);
      }
      return;
    }
  }
  for (int e = lane; e < MT * TEAMS * QUADS; e += 64) {
    const int r = e / (TEAMS * QUADS), team = (e / QUADS) % TEAMS, qq = e % QUADS;
    const int strip = team == 0 ? rd.y : rd.z;
    if (r >= M || strip < 0) continue;
    const f4_t sum = total(team, r, qq);
    h4_t y = {(_Float16)sum[0], (_Float16)sum[1], (_Float16)sum[2], (_Float16)sum[3]};
    if (st.epilogue == kEpilogueBias) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        y[c] = (_Float16)(static_cast<float>(y[c]) + static_cast<float>(bb[team * SW + 4 * qq + c]));
    }
    store(st.Y + static_cast<size_t>(r) * st.N + strip * SW + 4 * qq, y);
  }
}

template <int MT, int GROUP>
__global__ __launch_bounds__(kChainThreads) void chain_kernel(ChainArgs a) {
  using lds_ptr = __attribute__((address_space(3))) void*;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  // Round r's partials go to red[r & 1]: the staging wave may sum round r - 1
  // while round r is computed.
  constexpr int kRed = kComputeWaves * 64 * MT;
  __shared__ __attribute__((aligned(16))) float red[2 * kRed];
  __shared__ int s_abort;

  const uint32_t lane = threadIdx.x & 63u;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool stager = wave == kStagerWave;
  const const_ptr<ChainStage> stages = as_const(a.stages);
  const const_ptr<int4> rounds = as_const(a.rounds);
  const int r_begin = as_const(a.round_begin)[blockIdx.x];
  const int r_end = as_const(a.round_begin)[blockIdx.x + 1];

  unsigned char* const ring = lds;
  _Float16* const xbuf = reinterpret_cast<_Float16*>(lds + kRingBytes);
  unsigned char* const sbuf = reinterpret_cast<unsigned char*>(xbuf + 2 * a.xbuf_halves);
  unsigned char* const bbuf = sbuf + 2 * a.sbuf_bytes;

  // ---- compute waves: the weight feed ------------------------------------
  // A 1 KiB wave load is 256 / sw packed rows of a strip: lane l reads the
  // 16 bytes at column quad l % (sw / 4) of row l / (sw / 4), so the slot
  // holds the strip-major bytes whichever layout the words are in.
  int feed_r = r_begin - 1;  // round whose loads are being issued
  uint32_t feed_left = 0;    // this wave's loads left in it
  uint32_t feed_off = 0;     // scalar byte offset of the next one in the stage's Wt
  uint32_t feed_step = 0;    // scalar bytes from one load to the next
  uint32_t feed_lane = 0;    // this lane's byte offset within a load
  __amdgpu_buffer_rsrc_t feed_rs = make_rsrc(a.stages, 0);
  auto plan_round = [&](int r) {
    feed_r = r;
    feed_left = 0;
    if (r >= r_end) return;
    const int4 rd = rounds[r];
    const ChainStage st = stages[rd.x];
    const uint32_t waves = chain_waves(st.sw);
    const uint32_t team = wave / waves, wt = wave % waves;
    const int strip = team == 0 ? rd.y : rd.z;
    if (strip < 0) return;
    const uint32_t g0 = wt * st.groups / waves, g1 = (wt + 1) * st.groups / waves;
    const uint32_t chunk = GROUP * st.sw / 2;  // bytes of one quant group of a strip
    const uint32_t lpr = st.sw / 4;            // lanes a packed row of the strip takes
    feed_left = (g1 - g0) * chunk / kSlotBytes;
    feed_off = static_cast<uint32_t>(strip) * st.w_col + g0 * (GROUP / 8) * st.w_row;
    feed_step = (kSlotBytes / (4 * st.sw)) * st.w_row;
    feed_lane = lane / lpr * st.w_row + lane % lpr * 16u;
    feed_rs = make_rsrc(st.Wt, st.wbytes);
  };
  // The next load of the wave's sequence into `slot`; past the last round a
  // load that reads nothing keeps the count of loads in flight constant.
  auto issue = [&](uint32_t slot) {
    while (feed_left == 0 && feed_r < r_end) plan_round(feed_r + 1);
    const lds_ptr dst = (lds_ptr)(ring + (wave * kRing + slot) * kSlotBytes);
    const bool real = feed_left > 0;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(feed_rs, dst, 16, real ? feed_lane : kOutOfRange,
                                             real ? feed_off : 0u, 0, kPolicyNt);
    if (real) {
      feed_off += feed_step;
      --feed_left;
    }
  };
  uint32_t slot = 0;
  auto take = [&]() -> u4_t {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitRingOldest);
    const u4_t w = *reinterpret_cast<const u4_t*>(ring + (wave * kRing + slot) * kSlotBytes +
                                                   lane * 16u);
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // the slot is read before it is refilled
    __builtin_amdgcn_sched_barrier(0);
    issue(slot);
    slot = slot + 1 == kRing ? 0 : slot + 1;
    return w;
  };

  // ---- staging wave ---------------------------------------------------------
  int x_ready = -1, s_ready = -1;  // rounds whose activations / scales are staged
  bool aborted = false;
  auto after_done = [&](const ChainStage& st) {
    return st.after < 0 || __builtin_amdgcn_readfirstlane(load_coherent_u32(
                               a.counters + st.after)) >= st.after_items;
  };
  // Bounded wait for the stage this one reads from; false if it gave up.
  // The error flag (another workgroup gave up) is looked at every 64th poll,
  // so that a poll is one memory round trip.
  auto wait_after = [&](const ChainStage& st) {
    if (st.after < 0) return true;
    for (uint32_t n = 0;; ++n) {
      if (after_done(st)) return true;
      if ((n & 63u) == 63u || n >= kSpinCap) {
        const uint32_t err = __builtin_amdgcn_readfirstlane(load_coherent_u32(a.error));
        if (err != 0 || n >= kSpinCap) {
          if (lane == 0 && err == 0)
            __hip_atomic_store(a.error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          return false;
        }
      }
      __builtin_amdgcn_s_sleep(1);
    }
  };
  // Activation rows and bias slice of round r into buffer b (agent-coherent).
  auto stage_x = [&](int r, int b) {
    const int4 rd = rounds[r];
    const ChainStage st = stages[rd.x];
    _Float16* const xd = xbuf + b * a.xbuf_halves;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(st.X, st.xbytes);
    const uint32_t chunks = st.xbytes / 16;
    // Lanes past the end are masked off: an LDS-DMA lane writes its 16 bytes
    // even when its load is out of range.
    for (uint32_t blk = 0; blk * 64 < chunks; ++blk) {
      const uint32_t ch = blk * 64 + lane;
      if (ch < chunks)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(xd + blk * 512), 16, ch * 16u, 0,
                                                 0, kPolicySc1);
    }
    // Rows M .. MT - 1 of the block read as zeros.
    for (uint32_t e = static_cast<uint32_t>(a.M) * st.K / 8 + lane; e < MT * st.K / 8; e += 64)
      *reinterpret_cast<h8_t*>(xd + 8 * e) = h8_t{};
    if (st.epilogue == kEpilogueBias) {
      const uint32_t per = st.sw / 8;  // 16-byte chunks of one strip's biases
      const uint32_t team = lane / per, part = lane % per;
      const int strip = team == 0 ? rd.y : (team == 1 ? rd.z : -1);
      const __amdgpu_buffer_rsrc_t rb = make_rsrc(st.bias, st.N * 2u);
      if (strip >= 0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rb, (lds_ptr)(bbuf + b * kBiasBytes), 16,
            (static_cast<uint32_t>(strip) * st.sw + 8 * part) * 2u, 0, 0, kPolicySc1);
    }
  };
  // Scales of round r's strips into buffer b (read-only data: no waits),
  // strip-major in LDS whichever layout they are in: 16-byte chunk ch is
  // column piece ch % (sw / 8) of group row ch / (sw / 8).
  auto stage_scales = [&](int r, int b) {
    const int4 rd = rounds[r];
    const ChainStage st = stages[rd.x];
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(st.St, st.sbytes);
    const uint32_t chunks = st.s_strip / 16;
    const uint32_t ppr = st.sw / 8;  // 16-byte pieces of a scale row of the strip
    unsigned char* const sd = sbuf + b * a.sbuf_bytes;
#pragma unroll
    for (int team = 0; team < 2; ++team) {
      const int strip = team == 0 ? rd.y : rd.z;
      if (strip < 0) continue;
      const uint32_t base = static_cast<uint32_t>(strip) * st.s_col;
      for (uint32_t blk = 0; blk * 64 < chunks; ++blk) {
        const uint32_t ch = blk * 64 + lane;
        if (ch < chunks)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs, (lds_ptr)(sd + team * st.s_strip + blk * kSlotBytes), 16,
              base + ch / ppr * st.s_row + ch % ppr * 16u, 0, 0, kPolicyNt);
      }
    }
  };
  auto emit = [&](int r, int b) {
    const int4 rd = rounds[r];
    const ChainStage st = stages[rd.x];
    const _Float16* const bb = reinterpret_cast<const _Float16*>(bbuf + b * kBiasBytes);
    const float* const rb = red + b * kRed;
    switch (st.sw) {
      case 16: chain_emit<MT, 16>(st, rd, a.M, lane, rb, bb); break;
      case 32: chain_emit<MT, 32>(st, rd, a.M, lane, rb, bb); break;
      default: chain_emit<MT, 64>(st, rd, a.M, lane, rb, bb); break;
    }
    // Its LDS reads are done before the buffers are refilled.
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    if (st.signal) {
      wait_vm_stores();  // the outputs are visible before the count says so
      if (lane == 0)
        __hip_atomic_fetch_add(a.counters + rd.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (a.stamps != nullptr && lane == 0)
      __hip_atomic_fetch_max(a.stamps + rd.x, __builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  };

  if (stager) {
    if (lane == 0) {
      s_abort = 0;
      if (a.stamps != nullptr)
        __hip_atomic_fetch_min(a.stamps + a.n_stages, __builtin_amdgcn_s_memrealtime(),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kRing; ++i) issue(i);
  }

  // The outputs of round r - 1 are emitted before round r starts when another
  // stage waits for them (or nothing follows), else during round r, so that
  // the wait for their stores does not hold round r back.
  bool deferred = false;
  for (int r = r_begin;; ++r) {
    if (stager) {
      deferred = false;
      if (r > r_begin) {
        if (r < r_end && !stages[rounds[r - 1].x].signal)
          deferred = true;
        else
          emit(r - 1, (r - 1) & 1);
      }
      if (r < r_end && !aborted) {
        const ChainStage st = stages[rounds[r].x];
        if (x_ready != r) {
          aborted = !wait_after(st);
          if (!aborted) stage_x(r, r & 1);
        }
        if (s_ready != r) stage_scales(r, r & 1);
      }
      wait_vm_stores();
      if (lane == 0) s_abort = aborted ? 1 : 0;
    }
    lds_barrier();  // A(r): round r's activations and scales are in LDS
    if (s_abort != 0 || r >= r_end) {
      if (stager && deferred) emit(r - 1, (r - 1) & 1);
      break;
    }
    if (stager) {
      if (deferred) emit(r - 1, (r - 1) & 1);
      // Round r + 1's scales, and its activations if nothing is left to wait for.
      if (r + 1 < r_end) {
        stage_scales(r + 1, (r + 1) & 1);
        s_ready = r + 1;
        if (after_done(stages[rounds[r + 1].x])) {
          stage_x(r + 1, (r + 1) & 1);
          x_ready = r + 1;
        }
      }
    } else {
      const int4 rd = rounds[r];
      const ChainStage st = stages[rd.x];
      const int b = r & 1;
      const _Float16* xb = xbuf + b * a.xbuf_halves;
      const _Float16* sb = reinterpret_cast<const _Float16*>(sbuf + b * a.sbuf_bytes);
      float* const rb = red + b * kRed;
      const int team = wave / chain_waves(st.sw);
      const int strip = team == 0 ? rd.y : rd.z;
      if (strip >= 0) {
        switch (st.sw) {
          case 16:
            if constexpr (GROUP == 128) chain_round<MT, GROUP, 16>(st, strip, wave, lane, xb, sb, rb, take);
            break;
          case 32: chain_round<MT, GROUP, 32>(st, strip, wave, lane, xb, sb, rb, take); break;
          default: chain_round<MT, GROUP, 64>(st, strip, wave, lane, xb, sb, rb, take); break;
        }
      }
    }
    lds_barrier();  // B(r): round r's partials are in LDS
  }

  // Every LDS-DMA load of the workgroup lands before it ends.
  wait_vm_stores();
  lds_barrier();
  if (stager && lane == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev + 1 == gridDim.x) {
      // The last workgroup: every other one has finished with the counters.
      for (int s = 0; s < a.n_stages; ++s)
        __hip_atomic_store(a.counters + s, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.

struct Chain {
  int device = -1;
  int mt = 1;
  int group = 128;
  int grid = 0;
  int n_stages = 0;
  int n_rounds = 0;
  size_t lds = 0;
  void* mem = nullptr;  // descriptors, rounds, round_begin, control words
  ChainArgs args{};
  size_t ctrl_offset = 0;
};

hipError_t launch_chain(const Chain& c, hipStream_t stream) {
  const dim3 grid(c.grid), block(kChainThreads);
#define NIBBLE_CHAIN_CASE(MT, G)                                                     \
  if (c.mt == MT && c.group == G) {                                                 \
    chain_kernel<MT, G><<<grid, block, c.lds, stream>>>(c.args);                   \
    return hipGetLastError();                                                       \
  }
  NIBBLE_CHAIN_CASE(1, 128)
  NIBBLE_CHAIN_CASE(2, 128)
  NIBBLE_CHAIN_CASE(4, 128)
  NIBBLE_CHAIN_CASE(8, 128)
  NIBBLE_CHAIN_CASE(1, 64)
  NIBBLE_CHAIN_CASE(2, 64)
  NIBBLE_CHAIN_CASE(4, 64)
  NIBBLE_CHAIN_CASE(8, 64)
#undef NIBBLE_CHAIN_CASE
  return hipErrorInvalidValue;
}

const void* chain_kernel_fn(int mt, int group) {
#define NIBBLE_CHAIN_FN(MT, G) \
  if (mt == MT && group == G) return reinterpret_cast<const void*>(&chain_kernel<MT, G>);
  NIBBLE_CHAIN_FN(1, 128)
  NIBBLE_CHAIN_FN(2, 128)
  NIBBLE_CHAIN_FN(4, 128)
  NIBBLE_CHAIN_FN(8, 128)
  NIBBLE_CHAIN_FN(1, 64)
  NIBBLE_CHAIN_FN(2, 64)
  NIBBLE_CHAIN_FN(4, 64)
  NIBBLE_CHAIN_FN(8, 64)
#undef NIBBLE_CHAIN_FN
  return nullptr;
}

struct Range {
  uintptr_t lo = 0, hi = 0;  // [lo, hi)
  bool overlaps(const Range& o) const { return lo < o.hi && o.lo < hi; }
};
Range range_of(const void* p, size_t bytes) {
  Range r;
  r.lo = reinterpret_cast<uintptr_t>(p);
  r.hi = r.lo + bytes;
  return r;
}

// A round item's cost for the balancing: the bytes it streams plus a fixed
// allowance for a round's barriers, reduction and stores (about 1 us of one
// CU's share of HBM bandwidth).
constexpr double kRoundOverheadBytes = 32.0 * 1024;

// LDS of a chain: the weight ring, double-buffered activations (mt rows of
// the largest K), double-buffered scales (the largest round's), bias, and
// the static partials.  Returns the dynamic part; *total adds the static.
size_t chain_lds_bytes(int mt, int64_t kmax, size_t smax, size_t* total) {
  const size_t xbuf_halves = static_cast<size_t>(mt) * static_cast<size_t>(kmax);
  const size_t lds = kRingBytes + 2 * xbuf_halves * 2 + 2 * align_up(smax, 16) + 2 * kBiasBytes;
  *total = lds + 2 * sizeof(float) * kComputeWaves * 64 * mt + 16;
  return lds;
}

// Whether a one-stage chain of this weight has a plan: a strip-major plan
// whose team shape the chain runs, and LDS within the CU's.
bool chain_fits(int64_t M, int64_t K, int64_t N, int64_t G, int64_t SW) {
  StreamPlan p;
  if (SW <= 0 || N % SW != 0 || !plan_strip_major(M, K, N, G, SW, &p) ||
      p.waves != chain_waves(static_cast<int>(SW)))
    return false;
  const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const size_t smax = static_cast<size_t>(kComputeWaves / p.waves) * static_cast<size_t>(K / G * SW * 2);
  size_t total = 0;
  chain_lds_bytes(mt, K, smax, &total);
  return total <= kLdsMax;
}

}  // namespace

// Host-only plan construction, exposed for the C ABI below.
int chain_create(const nibble_chain_stage* stages, int64_t n, int64_t M, void* stream_,
                 void** out) {
  NIBBLE_CHECK(out != nullptr, "null output handle");
  *out = nullptr;
  NIBBLE_CHECK(stages != nullptr && n >= 1 && n <= 65535, "a chain needs 1..65535 stages, got %lld",
               (long long)n);
  NIBBLE_CHECK(M >= 1 && M <= 8, "a chain serves batches of 1..8 rows, got M=%lld", (long long)M);
  const int64_t G = stages[0].group_size;
  NIBBLE_CHECK(G == 64 || G == 128, "group_size must be 64 or 128, got %lld", (long long)G);
  const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  std::vector<ChainStage> desc(static_cast<size_t>(n));
  std::vector<int> items(static_cast<size_t>(n)), teams_of(static_cast<size_t>(n));
  std::vector<Range> in_x(n), in_b(n), outs(n), wts(n);
  int64_t kmax = 0;
  size_t smax = 0;
  const int64_t lim = int64_t(1) << 31;
  for (int64_t i = 0; i < n; ++i) {
    const nibble_chain_stage& s = stages[i];
    const int64_t K = s.K, N = s.N, SW = s.strip_cols;
    NIBBLE_CHECK(s.group_size == G, "stage %lld: every stage of a chain must share group_size %lld",
                 (long long)i, (long long)G);
    NIBBLE_CHECK(K > 0 && N > 0 && K % G == 0, "stage %lld: bad K=%lld / N=%lld for group_size %lld",
                 (long long)i, (long long)K, (long long)N, (long long)G);
    StreamPlan p;
    NIBBLE_CHECK(plan_strip_major(M, K, N, G, SW, &p) && (p.waves == 4 || p.waves == 8),
                 "stage %lld: no strip-major plan for K=%lld N=%lld strip_cols=%lld", (long long)i,
                 (long long)K, (long long)N, (long long)SW);
    NIBBLE_CHECK(p.waves == chain_waves(static_cast<int>(SW)), "stage %lld: plan mismatch",
                 (long long)i);
    NIBBLE_CHECK(s.epilogue == kEpilogueNone || s.epilogue == kEpilogueBias ||
                     s.epilogue == kEpilogueSwiglu,
                 "stage %lld: epilogue must be 0, 1 or 2, got %lld", (long long)i,
                 (long long)s.epilogue);
    NIBBLE_CHECK(s.epilogue != kEpilogueSwiglu || (SW >= 2 * kSwigluBlock && N % 32 == 0),
                 "stage %lld: swiglu needs strips of at least 32 columns", (long long)i);
    NIBBLE_CHECK(s.epilogue != kEpilogueBias || s.bias != nullptr, "stage %lld: null bias",
                 (long long)i);
    NIBBLE_CHECK(s.X != nullptr && s.Wt != nullptr && s.St != nullptr && s.Y != nullptr,
                 "stage %lld: null pointer", (long long)i);
    NIBBLE_CHECK(aligned(s.X, 16) && aligned(s.Wt, 16) && aligned(s.St, 16) && aligned(s.Y, 8) &&
                     (s.epilogue != kEpilogueBias || aligned(s.bias, 16)),
                 "stage %lld: X, Wt, St and bias need 16-byte alignment, Y 8-byte", (long long)i);
    NIBBLE_CHECK(s.after >= -1 && s.after < i, "stage %lld: `after` must name an earlier stage or be -1",
                 (long long)i);
    NIBBLE_CHECK(s.layout == 0 || s.layout == 1,
                 "stage %lld: layout must be 0 (strip-major) or 1 (packed), got %lld", (long long)i,
                 (long long)s.layout);
    const size_t wbytes = static_cast<size_t>(K / 8) * N * 4, sbytes = static_cast<size_t>(K / G) * N * 2;
    NIBBLE_CHECK(static_cast<int64_t>(wbytes) < lim && M * K * 2 < lim,
                 "stage %lld: operands beyond 32-bit offsets", (long long)i);
    ChainStage& d = desc[i];
    d.X = static_cast<const _Float16*>(s.X);
    d.Wt = static_cast<const uint32_t*>(s.Wt);
    d.St = static_cast<const _Float16*>(s.St);
    d.Y = static_cast<_Float16*>(s.Y);
    d.bias = s.epilogue == kEpilogueBias ? static_cast<const _Float16*>(s.bias) : nullptr;
    d.K = static_cast<uint32_t>(K);
    d.N = static_cast<uint32_t>(N);
    d.sw = static_cast<uint32_t>(SW);
    d.groups = static_cast<uint32_t>(K / G);
    d.w_strip = static_cast<uint32_t>(K / 8 * SW * 4);
    d.s_strip = static_cast<uint32_t>(K / G * SW * 2);
    const bool packed = s.layout == 1;
    d.w_col = packed ? static_cast<uint32_t>(SW * 4) : d.w_strip;
    d.w_row = static_cast<uint32_t>((packed ? N : SW) * 4);
    d.s_col = packed ? static_cast<uint32_t>(SW * 2) : d.s_strip;
    d.s_row = static_cast<uint32_t>((packed ? N : SW) * 2);
    d.pad = 0;
    d.wbytes = static_cast<uint32_t>(wbytes);
    d.sbytes = static_cast<uint32_t>(sbytes);
    d.xbytes = static_cast<uint32_t>(M * K * 2);
    d.epilogue = static_cast<uint32_t>(s.epilogue);
    d.after = static_cast<int32_t>(s.after);
    d.after_items = 0;
    d.signal = 0;
    const int teams = kComputeWaves / p.waves;
    teams_of[i] = teams;
    items[i] = static_cast<int>(ceil_div(N / SW, teams));
    kmax = std::max(kmax, K);
    smax = std::max(smax, static_cast<size_t>(teams) * d.s_strip);
    const int64_t nout = s.epilogue == kEpilogueSwiglu ? N / 2 : N;
    in_x[i] = range_of(s.X, static_cast<size_t>(M * K * 2));
    in_b[i] = s.epilogue == kEpilogueBias ? range_of(s.bias, static_cast<size_t>(N * 2)) : Range();
    outs[i] = range_of(s.Y, static_cast<size_t>(M * nout * 2));
    wts[i] = range_of(s.Wt, wbytes);
  }
  // Dependencies: whatever a stage reads that another stage writes must be
  // ordered by the `after` links (reads after the write, writes after the
  // reads), so no two stages that may run at once touch the same bytes.
  std::vector<std::vector<char>> anc(static_cast<size_t>(n), std::vector<char>(static_cast<size_t>(n), 0));
  for (int64_t i = 0; i < n; ++i)
    for (int64_t j = stages[i].after; j >= 0; j = stages[j].after) anc[i][j] = 1;
  for (int64_t i = 0; i < n; ++i) {
    NIBBLE_CHECK(!outs[i].overlaps(in_x[i]) && !outs[i].overlaps(in_b[i]),
                 "stage %lld: output overlaps its own inputs", (long long)i);
    for (int64_t j = 0; j < n; ++j) {
      NIBBLE_CHECK(!outs[j].overlaps(wts[i]) &&
                       !outs[j].overlaps(range_of(stages[i].St, desc[i].sbytes)),
                   "stage %lld writes stage %lld's weights", (long long)j, (long long)i);
      if (j == i) continue;
      const bool reads = outs[j].overlaps(in_x[i]) || outs[j].overlaps(in_b[i]);
      const bool writes = outs[j].overlaps(outs[i]);
      if (j < i) {
        NIBBLE_CHECK(!(reads || writes) || anc[i][j],
                     "stage %lld reads or writes what stage %lld writes without waiting for it "
                     "(set `after` to it or to a stage that waits for it)",
                     (long long)i, (long long)j);
      } else {
        NIBBLE_CHECK(!reads || anc[j][i],
                     "stage %lld overwrites what stage %lld reads without waiting for it",
                     (long long)j, (long long)i);
      }
    }
  }
  for (int64_t i = 0; i < n; ++i)
    if (desc[i].after >= 0) {
      desc[i].after_items = static_cast<uint32_t>(items[desc[i].after]);
      desc[desc[i].after].signal = 1;
    }

  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  int cus = 0;
  NIBBLE_HIP(cu_count(dev, &cus));
  const size_t xbuf_halves = static_cast<size_t>(mt) * static_cast<size_t>(kmax);
  const size_t sbuf = align_up(smax, 16);
  size_t lds_total = 0;
  const size_t lds = chain_lds_bytes(mt, kmax, smax, &lds_total);
  NIBBLE_CHECK(lds_total <= kLdsMax,
               "chain needs %zu bytes of LDS (M=%lld, largest K=%lld); the limit is %zu",
               lds_total, (long long)M, (long long)kmax, kLdsMax);
  const void* fn = chain_kernel_fn(mt, static_cast<int>(G));
  int per_cu = 0;
  NIBBLE_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kChainThreads, lds));
  if (per_cu < 1) return fail(NIBBLE_ERR_UNSUPPORTED, "chain kernel does not fit a CU");
  // One workgroup per CU: every workgroup must be resident for the waits.
  const int grid = cus;

  // Rounds, stages in order, so every workgroup's list is in stage order.
  // Within a stage every workgroup takes the same number of round items, up
  // to one more: a stage that others wait for ends with its slowest
  // workgroup.  The extra items go to the workgroups with the least work so
  // far (bytes plus a per-round allowance), which balances the whole chain.
  std::vector<std::vector<int4>> lists(static_cast<size_t>(grid));
  std::vector<double> load(static_cast<size_t>(grid), 0.0);
  std::vector<int> order(static_cast<size_t>(grid));
  for (int64_t i = 0; i < n; ++i) {
    const int strips = static_cast<int>(desc[i].N / desc[i].sw), teams = teams_of[i];
    const int base = items[i] / grid, extra = items[i] % grid;
    for (int w = 0; w < grid; ++w) order[w] = w;
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return load[x] < load[y]; });
    int k = 0;
    for (int pos = 0; pos < grid; ++pos) {
      const int w = order[pos];
      const int take = base + (pos < extra ? 1 : 0);
      for (int t = 0; t < take; ++t, ++k) {
        int4 item;
        item.x = static_cast<int>(i);
        item.y = k * teams;
        item.z = teams == 2 && k * teams + 1 < strips ? k * teams + 1 : -1;
        item.w = 0;
        const int used = item.z >= 0 ? 2 : 1;
        lists[w].push_back(item);
        load[w] += used * (desc[i].w_strip + desc[i].s_strip) + kRoundOverheadBytes;
      }
    }
  }
  std::vector<int> begin(static_cast<size_t>(grid) + 1, 0);
  std::vector<int4> rounds;
  for (int w = 0; w < grid; ++w) {
    begin[w] = static_cast<int>(rounds.size());
    rounds.insert(rounds.end(), lists[w].begin(), lists[w].end());
  }
  begin[grid] = static_cast<int>(rounds.size());

  const size_t off_stages = 0;
  const size_t off_rounds = align_up(off_stages + desc.size() * sizeof(ChainStage), 256);
  const size_t off_begin = align_up(off_rounds + rounds.size() * sizeof(int4), 256);
  const size_t off_ctrl = align_up(off_begin + begin.size() * sizeof(int), 256);
  const size_t ctrl_words = static_cast<size_t>(n) + 2;
  const size_t total = align_up(off_ctrl + ctrl_words * 4, 256);
  std::vector<unsigned char> host(total, 0);
  std::memcpy(host.data() + off_stages, desc.data(), desc.size() * sizeof(ChainStage));
  std::memcpy(host.data() + off_rounds, rounds.data(), rounds.size() * sizeof(int4));
  std::memcpy(host.data() + off_begin, begin.data(), begin.size() * sizeof(int));

  Chain* c = new (std::nothrow) Chain();
  if (c == nullptr) return fail(NIBBLE_ERR_UNSUPPORTED, "out of host memory");
  hipError_t e = hipMalloc(&c->mem, total);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "hipMalloc (chain plan)");
  }
  e = hipMemcpy(c->mem, host.data(), total, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(c->mem);
    delete c;
    return hip_fail(e, "hipMemcpy (chain plan)");
  }
  unsigned char* base = static_cast<unsigned char*>(c->mem);
  c->device = dev;
  c->mt = mt;
  c->group = static_cast<int>(G);
  c->grid = grid;
  c->n_stages = static_cast<int>(n);
  c->n_rounds = static_cast<int>(rounds.size());
  c->lds = lds;
  c->ctrl_offset = off_ctrl;
  ChainArgs& a = c->args;
  a.stages = reinterpret_cast<const ChainStage*>(base + off_stages);
  a.rounds = reinterpret_cast<const int4*>(base + off_rounds);
  a.round_begin = reinterpret_cast<const int*>(base + off_begin);
  a.counters = reinterpret_cast<uint32_t*>(base + off_ctrl);
  a.done = a.counters + n;
  a.error = a.counters + n + 1;
  a.stamps = nullptr;
  a.M = static_cast<int>(M);
  a.n_stages = static_cast<int>(n);
  a.xbuf_halves = static_cast<uint32_t>(xbuf_halves);
  a.sbuf_bytes = static_cast<uint32_t>(sbuf);
  *out = c;
  return NIBBLE_OK;
}

}  // namespace nibble

using namespace nibble;

extern "C" int64_t nibble_chain_strip_cols(int64_t K, int64_t N, int64_t group_size, int64_t M) {
  // A chain round costs a fixed allowance (barriers, partial sums, stores)
  // besides its bytes, so fewer, wider strips win: the widest of 64 and 32
  // columns the chain has a plan for, else the launches' width.  Measured on
  // MI355X, the 8B step as one chain: 0.585 -> 0.552 ms per token with o and
  // down in 32-column strips instead of 16 (64-column o and q|k|v: the same;
  // 64-column down does not fit the LDS); at one GPU's share of an 8-way
  // split 0.124 ms with every weight in 32-column strips, 0.085 in 64.
  const int64_t base = strip_major_cols(K, N, group_size);
  if (base == 0 || M < 1 || M > 8) return 0;
  for (const int64_t sw : {int64_t(64), int64_t(32), base})
    if (chain_fits(M, K, N, group_size, sw)) return sw;
  return 0;
}

extern "C" int nibble_chain_create(const nibble_chain_stage* stages, int64_t n_stages, int64_t M,
                                   void* stream, void** chain) {
  const int rc = chain_create(stages, n_stages, M, stream, chain);
  return rc == NIBBLE_OK ? ok() : rc;
}

extern "C" int nibble_chain_run(void* chain, void* timestamps, void* stream_) {
  NIBBLE_CHECK(chain != nullptr, "null chain");
  Chain* c = static_cast<Chain*>(chain);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  NIBBLE_CHECK(dev == c->device, "chain was built for device %d, stream is on device %d",
               c->device, dev);
  NIBBLE_CHECK(timestamps == nullptr || aligned(timestamps, 8), "misaligned timestamps");
  Chain run = *c;
  run.args.stamps = static_cast<unsigned long long*>(timestamps);
  const hipError_t e = launch_chain(run, stream);
  if (e != hipSuccess) return hip_fail(e, "chain kernel launch");
  return ok();
}

extern "C" int nibble_chain_check(void* chain, void* stream_) {
  NIBBLE_CHECK(chain != nullptr, "null chain");
  Chain* c = static_cast<Chain*>(chain);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  NIBBLE_HIP(hipStreamSynchronize(stream));
  uint32_t err = 0;
  NIBBLE_HIP(hipMemcpy(&err, c->args.error, sizeof(err), hipMemcpyDeviceToHost));
  if (err != 0) {
    const uint32_t zero = 0;
    NIBBLE_HIP(hipMemcpy(c->args.error, &zero, sizeof(zero), hipMemcpyHostToDevice));
    return fail(NIBBLE_ERR_HIP,
                "a chain run gave up waiting for a stage (another workgroup was not resident "
                "or did not finish); its outputs are incomplete");
  }
  return ok();
}

extern "C" int64_t nibble_chain_info(void* chain, int64_t what) {
  if (chain == nullptr) return -1;
  const Chain* c = static_cast<const Chain*>(chain);
  switch (what) {
    case 0: return c->grid;
    case 1: return c->n_rounds;
    case 2: return static_cast<int64_t>(c->lds);
    case 3: return c->n_stages;
    default: return -1;
  }
}

extern "C" int nibble_chain_destroy(void* chain) {
  if (chain == nullptr) return ok();
  Chain* c = static_cast<Chain*>(chain);
  const hipError_t e = hipFree(c->mem);
  delete c;
  if (e != hipSuccess) return hip_fail(e, "hipFree (chain plan)");
  return ok();
}
