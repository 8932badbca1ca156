// vmrt_calibrate: measured costs for the scheduler's work model.
//
// The reference times one small program per tile-op family at two tile counts
// and takes the slope as microseconds per tile, written to a JSON cost table
// that the lowering subprocess reads through PJRT_OCL_COST_TABLE
// (runtime.cc:2360-2517; scheduler.py:135-153).  This build measures the same
// four per-tile costs (one lane, so the slope is what one CU pays per tile) and
// the terms of its own phase model: the latency of a tile, the bandwidth one
// lane streams at when every lane streams, and the grid barrier's cost and its
// growth with the lane count.  Every program is built here as VMProgram v3
// bytes (schedule sections only, like the reference's runtime_test programs)
// and runs through the public C ABI.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/vmrt.h"
#include "vm_abi.h"

namespace {

using namespace vm;

// A schedule-only VMProgram v3 writer.
struct Builder {
  struct Buf { uint64_t off, size; uint32_t dt; };
  std::vector<Buf> bufs;
  std::vector<int32_t> aux;
  std::vector<Task> tasks;
  std::vector<std::vector<Entry>> lanes;
  uint64_t arena = 0;

  explicit Builder(uint32_t n_lanes) : lanes(n_lanes) {}

  uint32_t buf(uint64_t elems, uint32_t dt) {
    const uint64_t size = elems * (dt == DT_BF16 || dt == DT_F16 ? 2 : 4);
    bufs.push_back({arena, size, dt});
    arena += (std::max<uint64_t>(size, 64) + 63) / 64 * 64;
    return uint32_t(bufs.size() - 1);
  }
  uint32_t task(uint32_t top, uint32_t dt, uint32_t adt, uint32_t dst, uint32_t a, uint32_t b,
                std::initializer_list<uint32_t> p) {
    Task t{};
    t.tile_op = top | dt << 8 | adt << 16;
    t.dst = dst;
    t.a = a;
    t.b = b;
    int k = 0;
    for (uint32_t v : p) t.p[k++] = v;
    tasks.push_back(t);
    return uint32_t(tasks.size() - 1);
  }
  void tiles(uint32_t lane, uint32_t task_id, uint32_t lo, uint32_t hi) {
    lanes[lane].push_back(Entry{task_id, lo, hi, 0xFFFFFFFFu, 0, 0xFFFFFFFFu, 0, 0});
  }
  // tiles [0, n) split evenly over every lane
  void spread(uint32_t task_id, uint32_t n) {
    const uint32_t L = uint32_t(lanes.size());
    for (uint32_t l = 0; l < L; ++l) {
      const uint32_t lo = uint32_t(uint64_t(n) * l / L), hi = uint32_t(uint64_t(n) * (l + 1) / L);
      if (hi > lo) tiles(l, task_id, lo, hi);
    }
  }
  void barrier() {
    for (auto& s : lanes) s.push_back(Entry{0xFFFFFFFEu, 0, 0, 0xFFFFFFFFu, 0, 0xFFFFFFFFu, 0, 0});
  }

  std::vector<uint8_t> bytes() const {
    std::vector<uint8_t> out;
    auto put = [&](const void* p, size_t n) {
      const uint8_t* b = static_cast<const uint8_t*>(p);
      out.insert(out.end(), b, b + n);
    };
    auto u32 = [&](uint32_t v) { put(&v, 4); };
    auto pad8 = [&] { out.resize((out.size() + 7) / 8 * 8, 0); };
    // header: magic, version, n_buffers, n_instrs, n_consts, main_len, n_inputs,
    // n_outputs, n_aux, pad, arena_bytes
    for (uint32_t v : {0x314D5056u, 3u, uint32_t(bufs.size()), 0u, 0u, 0u, 0u, 0u, uint32_t(aux.size()), 0u}) u32(v);
    const uint64_t ab = std::max<uint64_t>(arena, 64);
    put(&ab, 8);
    for (const Buf& b : bufs) {
      put(&b.off, 8);
      put(&b.size, 8);
      u32(b.dt);
      u32(0);
    }
    // no io maps or shapes; aux; no consts; no instructions
    if (!aux.empty()) put(aux.data(), aux.size() * 4);
    pad8();
    size_t n_entries = 0;
    for (auto& s : lanes) n_entries += s.size();
    for (uint32_t v : {uint32_t(tasks.size()), uint32_t(n_entries), 0u, uint32_t(lanes.size())}) u32(v);
    put(tasks.data(), tasks.size() * sizeof(Task));
    uint32_t off = 0;
    for (auto& s : lanes) {
      for (uint32_t v : {off, uint32_t(s.size()), uint32_t(s.size()), 0u}) u32(v);
      off += uint32_t(s.size());
    }
    for (auto& s : lanes) put(s.data(), s.size() * sizeof(Entry));
    return out;
  }
};

struct Timer {
  vmrt_runtime* rt;
  std::string* err;

  // best over 3 rounds of `reps` back-to-back launches, microseconds per launch
  double time(const Builder& b, uint32_t ew_ts, int reps) {
    const std::vector<uint8_t> blob = b.bytes();
    vmrt_program* p = nullptr;
    char e[1024];
    if (vmrt_load(rt, blob.data(), blob.size(), ew_ts, 0, &p, e, sizeof e) != VMRT_OK) {
      *err = e;
      return -1.0;
    }
    void *t0 = nullptr, *t1 = nullptr;
    vmrt_event_create(rt, &t0);
    vmrt_event_create(rt, &t1);
    double best = 1e30;
    bool ok = vmrt_execute(p, nullptr, 0, nullptr, 0, e, sizeof e) == VMRT_OK;   // warm-up
    for (int round = 0; ok && round < 3; ++round) {
      vmrt_event_record(rt, t0, nullptr);
      for (int r = 0; ok && r < reps; ++r) ok = vmrt_enqueue(p, nullptr, 0, nullptr, 0, nullptr, e, sizeof e) == VMRT_OK;
      vmrt_event_record(rt, t1, nullptr);
      float ms = 0.f;
      ok = ok && vmrt_event_elapsed_ms(t0, t1, &ms) == VMRT_OK;
      best = std::min(best, 1e3 * double(ms) / reps);
    }
    ok = ok && vmrt_program_status(p, e, sizeof e) == VMRT_OK;
    if (!ok) *err = e;
    vmrt_event_destroy(t0);
    vmrt_event_destroy(t1);
    vmrt_unload(p);
    return ok ? best : -1.0;
  }
};

// One lane, `tiles` tiles of a family; ew_ts elements per elementwise tile.
Builder family(int fam, uint32_t tiles, uint32_t ew_ts, uint32_t mma_t) {
  Builder b(1);
  const uint64_t n = uint64_t(tiles) * ew_ts;
  switch (fam) {
    case 0: {   // elementwise multiply, f32
      const uint32_t x = b.buf(n, DT_F32), y = b.buf(n, DT_F32), d = b.buf(n, DT_F32);
      b.tiles(0, b.task(TOP_EW, DT_F32, DT_F32, d, x, y, {SUB_MUL, uint32_t(n), 0, 0}), 0, tiles);
      break;
    }
    case 1: {   // matmul tile, bf16 operands, f32 accumulate: M = tiles * T, N = T, K = 256
      const uint32_t M = tiles * mma_t, N = mma_t, K = 256;
      const uint32_t A = b.buf(uint64_t(M) * K, DT_BF16), B = b.buf(uint64_t(K) * N, DT_BF16),
                     C = b.buf(uint64_t(M) * N, DT_F32);
      b.tiles(0, b.task(TOP_MMA, DT_F32, DT_BF16, C, A, B, {M, N, K, 1}), 0, tiles);
      break;
    }
    case 2: {   // partial sums, one chunk of ew_ts per tile
      const uint32_t x = b.buf(n, DT_F32), parts = b.buf(tiles, DT_F32);
      b.tiles(0, b.task(TOP_RED_PART, DT_F32, DT_F32, parts, x, x, {uint32_t(n), ew_ts, 0}), 0, tiles);
      break;
    }
    default: {  // identity strided gather, rank 1
      const uint32_t x = b.buf(n, DT_F32), d = b.buf(n, DT_F32);
      b.aux = {1, int32_t(n), 1, 0};
      b.tiles(0, b.task(TOP_GATHER, DT_F32, DT_F32, d, x, x, {0, uint32_t(n)}), 0, tiles);
      break;
    }
  }
  return b;
}

// `count` phases, each a grid barrier, optionally after one small elementwise
// tile per lane (64 elements: its time is the tile's fixed latency)
Builder barriers(uint32_t lanes, uint32_t count, bool with_tile = false) {
  Builder b(lanes);
  uint32_t t = 0;
  if (with_tile) {
    const uint64_t n = uint64_t(lanes) * 64;
    const uint32_t x = b.buf(n, DT_F32), d = b.buf(n, DT_F32);
    t = b.task(TOP_EW, DT_F32, DT_F32, d, x, x, {SUB_EXP, uint32_t(n), 0, 0});
  }
  for (uint32_t k = 0; k < count; ++k) {
    if (with_tile)
      for (uint32_t l = 0; l < lanes; ++l) b.tiles(l, t, l, l + 1);
    b.barrier();
  }
  return b;
}

// one lane, `tiles` matmul tiles of the fast path: 256 x 256 outputs, K = 1024, bf16
Builder mma_fast(uint32_t tiles) {
  Builder b(1);
  const uint32_t M = 256 * tiles, N = 256, K = 1024;
  const uint32_t A = b.buf(uint64_t(M) * K, DT_BF16), B = b.buf(uint64_t(K) * N, DT_BF16),
                 C = b.buf(uint64_t(M) * N, DT_F32);
  b.tiles(0, b.task(TOP_MMA, DT_F32, DT_BF16, C, A, B, {M, N, K, 1u | (3u << 24)}), 0, tiles);
  return b;
}

// every lane streams its share of a copy of `n` floats (read + write)
Builder stream(uint32_t lanes, uint64_t n, uint32_t ew_ts) {
  Builder b(lanes);
  const uint32_t x = b.buf(n, DT_F32), d = b.buf(n, DT_F32);
  b.spread(b.task(TOP_EW, DT_F32, DT_F32, d, x, x, {SUB_COPY, uint32_t(n), 0, 0}), uint32_t((n + ew_ts - 1) / ew_ts));
  return b;
}

}  // namespace

extern "C" int vmrt_calibrate(vmrt_runtime* rt, char* json, size_t cap, char* err, size_t errlen) {
  auto fail = [&](const std::string& m) {
    if (err && errlen) std::snprintf(err, errlen, "calibration: %s", m.c_str());
    return VMRT_INTERNAL;
  };
  if (!rt || !json || !cap) return VMRT_INVALID_ARGUMENT;
  vmrt_device_info I;
  vmrt_device_info_get(rt, &I);
  std::string msg;
  Timer T{rt, &msg};
  // per-tile cost of each family on one lane (ew, mma, reduce, gather: the
  // reference's four keys, written below): slope between t and 2t tiles
  const uint32_t t_lo[4] = {32, 8, 32, 32};
  double us[4];
  for (int f = 0; f < 4; ++f) {
    const double a = T.time(family(f, t_lo[f], I.ew_ts, I.mma_t), I.ew_ts, 20);
    const double b = T.time(family(f, 2 * t_lo[f], I.ew_ts, I.mma_t), I.ew_ts, 20);
    if (a < 0 || b < 0) return fail(msg);
    us[f] = std::max(0.01, (b - a) / t_lo[f]);
  }
  // grid barrier: slope over the barrier count at the full and the half lane count
  const uint32_t L = I.n_lanes, H = std::max(1u, I.n_lanes / 2);
  // tile latency: what one small tile per lane adds to a phase
  const double pa = T.time(barriers(L, 64, true), 64, 10), pb = T.time(barriers(L, 64), 64, 10);
  if (pa < 0 || pb < 0) return fail(msg);
  const double tile_us = std::max(0.01, (pa - pb) / 64);
  // MFMA rate of one lane on the matmul fast path
  const double ma = T.time(mma_fast(2), I.ew_ts, 10), mb = T.time(mma_fast(4), I.ew_ts, 10);
  if (ma < 0 || mb < 0) return fail(msg);
  const double lane_mma_tflops = mb > ma ? 2.0 * 256 * 256 * 1024 * 2 / ((mb - ma) * 1e6) : 0.0;
  double bar[2];
  const uint32_t lane_counts[2] = {L, H};
  for (int k = 0; k < 2; ++k) {
    const double a = T.time(barriers(lane_counts[k], 64), I.ew_ts, 10);
    const double b = T.time(barriers(lane_counts[k], 128), I.ew_ts, 10);
    if (a < 0 || b < 0) return fail(msg);
    bar[k] = std::max(0.01, (b - a) / 64);
  }
  const double per_lane = L > H ? std::max(0.0, (bar[0] - bar[1]) / (L - H)) : 0.0;
  const double bar0 = std::max(0.01, bar[0] - per_lane * L);
  // streaming bandwidth per lane with every lane streaming: slope between two copy sizes
  const uint64_t n1 = uint64_t(16) << 20, n2 = uint64_t(32) << 20;   // floats
  const double sa = T.time(stream(L, n1, I.ew_ts), I.ew_ts, 5), sb = T.time(stream(L, n2, I.ew_ts), I.ew_ts, 5);
  if (sa < 0 || sb < 0) return fail(msg);
  const double lane_gbs = (sb > sa) ? double(n2 - n1) * 8.0 / ((sb - sa) * 1e3) / L : 0.0;
  const int w = std::snprintf(
      json, cap,
      "{\"ew_tile_us\": %.4f, \"mma_tile_us\": %.4f, \"reduce_tile_us\": %.4f, \"gather_tile_us\": %.4f, "
      "\"tile_us\": %.4f, \"barrier_us\": %.4f, \"barrier_us_per_lane\": %.6f, \"lane_gbs\": %.3f, "
      "\"lane_mma_tflops\": %.4f, \"lanes\": %u, \"ew_ts\": %u, \"mma_t\": %u, \"device\": \"%s %s\"}",
      us[0], us[1], us[2], us[3], tile_us, bar0, per_lane, lane_gbs, lane_mma_tflops, L, I.ew_ts,
      I.mma_t, I.name, I.arch);
  if (w < 0 || size_t(w) >= cap) return fail("JSON buffer too small");
  return VMRT_OK;
}
