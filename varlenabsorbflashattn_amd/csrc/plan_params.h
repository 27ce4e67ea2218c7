// Tile sizes and key-split policy shared by the planner and the kernels.
#pragma once
#include <cstdint>

namespace vafa {

// Varlen: a forward / dQ workgroup covers one query tile (32 rows per wave)
// and a dK/dV workgroup one key tile (32 keys per wave).  The planner picks
// each per call between kVarlenTile (4-wave workgroups) and kVarlenWideTile
// (8-wave workgroups, D <= 128 only: at D=256 one wave per SIMD holds the
// registers); the fused K-major pass always uses kVarlenTile keys.
constexpr int kVarlenTile = 128;
constexpr int kVarlenWideTile = 256;
// Absorb: a forward workgroup covers up to kAbsorbRows (token, head) rows;
// a dX workgroup covers up to kAbsorbKTile keys of one sample (four 128-key
// sub-tiles on the matrix-core path).
constexpr int kAbsorbRows = 64;
constexpr int kAbsorbKTile = 512;

struct SplitPolicy {
  // Query tiles with at most `decode_rows` rows against >= decode_min_keys
  // keys are split into clamp(ceil(Lk/decode_chunk), min, max) chunks.
  int64_t decode_rows, decode_min_keys, decode_chunk, decode_min_split, decode_max_split;
  // Any other tile is split into ceil(Lk/long_chunk) chunks once
  // Lk > long_threshold (fa/interface.py:46-57 uses 4096 / 4096).
  int64_t long_threshold, long_chunk;
  int64_t align;          // chunk lengths are multiples of this many keys
  int64_t item_overhead;  // fixed per-item cost (keys-equivalent) for LPT
};

constexpr SplitPolicy kVarlenPolicy{16, 1024, 2048, 4, 16, 4096, 4096, 64, 64};
// Absorb: long_chunk is the smallest key chunk; the planner raises chunk and
// threshold with the launch's total work (see vafa_plan_absorb).
constexpr SplitPolicy kAbsorbPolicy{0, 1 << 30, 1024, 1, 16, 1024, 1024, 64, 32};
// Resident absorb forward workgroups on the MI355X (256 CUs x 3), and the
// multiple of the average keys per workgroup that a key range may hold
// before it is split (measured: splitting configs[4]'s <= 8192-key samples
// into 1024-key chunks cost 10%, configs[3]'s <= 2000-key samples at 1024
// keys 4%).
constexpr int64_t kAbsorbSlots = 768;
constexpr int64_t kAbsorbSplitSlack = 3;

// Varlen backward, fused K-major path (dQ, dK, dV in one kernel, fp32 dQ
// partials per key chunk summed in order): segments with at most kFusedMaxQ
// queries and at least kFusedMinK keys, at head dims up to kFusedMaxD.  Each
// chunk writes Lq*D*4 bytes of partial dQ (plus the read back in the sum) and
// saves the second read of its K/V rows that the query-major dQ kernel makes.
// Measured on the MI355X with one 128-key tile per item (64 segments x 8192
// keys, backward
// ms, two-kernel vs fused): H=4 D=64 Lq=1/8/16: 0.447/0.440/0.451 vs
// 0.379/0.387/0.394; Lq=32 0.443 vs 0.440; Lq=48/64 0.487/0.472 vs
// 0.519/0.561.  At D=128 the fused kernel holds one workgroup per CU (256
// VGPRs + 225 AGPRs, 117 KB of LDS) and lost at every Lq (1.57-1.59 vs
// 1.65-1.95 ms at H=8), so it serves D <= 64 only.
constexpr int kFusedMaxQ = 16;
constexpr int kFusedMinK = 1;
constexpr int kFusedMaxD = 64;
// A fused item walks up to kFusedTiles 128-key tiles of one segment (the
// query block staged once, dQ summed over the chunk in registers).  Measured
// on the MI355X, backward ms for 1 / 2 / 3 / 4 tiles per item: 64 x 16 queries
// x 8192 keys (H=4, D=64) 0.667 / 0.666 / 0.607 / 0.750; 256 x 8 x 2048 keys
// 0.644 / 0.663 / 0.638 / 0.780; 32 x 1 x 32768 keys (H=8) 2.47 / 2.41 /
// 2.37 / 2.44.
constexpr int kFusedTiles = 3;

// Workgroups are dispatched round-robin over this many XCDs (one L2 each):
// workgroup i runs on XCD i % kXcds.
constexpr int kXcds = 8;

// Absorb dX: a segment with at most this many (token, head) rows keeps all of
// them resident in one workgroup (absorb_dx_res_kernel); longer segments are
// streamed in 32-row blocks (absorb_dx_kernel).
constexpr int kDxResidentRows = 64;

}  // namespace vafa
