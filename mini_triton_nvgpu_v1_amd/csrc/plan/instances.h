// The gfx950 kernel instances compiled into libtb_gfx950.so, as host data:
// the tile lists of kernels/gemm_tiles.h in every output mode (plain) and in
// the whole-result modes (fused epilogue steps), plus the 16x16x32
// instances. KernelConfig legality and tb-lower-pipeline-to-gfx950 consult
// this table, so the plan refuses a configuration with no kernel and the
// lowering never names one that does not exist. tb-opt carries it without
// the kernels (`tb-opt --list-instances`).
#pragma once

#include "tb_gfx950.h"

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace tb {

// Output modes of an instance (the kernels' OutMode).
enum InstanceOut : int {
  kInstOutF16 = 0,        // C(f16) = A*B
  kInstOutF32Partial = 1, // f32 store: split-K partial plane, or plain f32 C
  kInstOutF32Accum = 2,   // C(f32) += A*B
  kInstOutF32Atomic = 3,  // C(f32) += partial sums with atomics
};

struct InstanceKey {
  int64_t bm = 0, bn = 0, bk = 0, wgm = 0, wgn = 0;
  int out = 0;
  int64_t stages = 0;
  int epi = 0;  // 1: the fused epilogue steps are compiled in
  int mfma = 0; // TB_MFMA_*
  bool operator<(const InstanceKey &o) const;
  bool operator==(const InstanceKey &o) const;
};

const std::vector<InstanceKey> &gfx950Instances();
bool hasGfx950Instance(const InstanceKey &k);
// tb_gemm_gfx950_{BM}x{BN}x{BK}_w{WGM}x{WGN}_s{S}_out{OUT}[_16x16x32][_epi]
std::string instanceName(const InstanceKey &k);
// The instance a flattened configuration binds: the output mode follows
// from C's type, C's initialisation and the reduction; split-K partials take
// the fused steps in the reduction, so they bind the plain instance.
InstanceKey instanceKeyOf(const tb_gemm_config &c);
// The output mode instanceKeyOf binds, from the facts that decide it (the
// plans state them before the lowering flattens them into tb_gemm_config).
int instanceOutOf(bool splitK, bool atomicReduction, bool f16C, bool loadC);
// How an instance issues its direct-to-LDS loads, and the s_waitcnt depths
// that follow (the kernel's GemmTile slot geometry, restated on the host):
//  * "slot_spread": wave tiles of 4+ MFMAs per k step; the k-tile is cut
//    into MFMA slots and a refill's loads are spread one per slot over
//    `refillSpreadSlots` slots from the barrier on; the prologue issues
//    k-tiles 0 .. S-2 whole and the first `prologueTailLoads` loads of k-tile
//    S-1 (those a refill issues before the next barrier);
//  * "burst": smaller wave tiles; a refill is issued whole right after the
//    barrier, and the prologue issues all S k-tiles;
//  * "exact_tile_slots": the hand-scheduled 16x16x32 instance (k-tiles 0 and
//    1 whole in the prologue; every barrier waits for all loads and LDS
//    reads);
//  * "tile16_slots": the 16x16x32 loop of the other tiles (all S k-tiles
//    whole in the prologue; each barrier waits for the next k-tile and, with
//    lgkmcnt(0), for the wave's LDS reads; the refill of the freed stage is
//    spread over `refillSpreadSlots` MFMA slots);
//  * "producer_waves": the f32-partial tiles of TBK_PRODUCER_TILES, whose
//    workgroup adds `loaderWaves` waves that only issue the loads: they issue
//    all S k-tiles in the prologue and, at each barrier, wait for the next
//    k-tile only (vmcnt (S-1) and (S-2) loads-per-thread), then refill the
//    stage the barrier freed whole.
// vmcnt at the prologue wait = (S-2) loads-per-thread + prologueTailLoads,
// vmcnt at the per-k-tile barrier = (S-2) loads-per-thread; lgkmcnt -1 = none.
struct InstanceSchedule {
  std::string issue;
  int64_t loadsPerThread = 0, prologueTailLoads = 0, refillSpreadSlots = 0;
  int64_t vmPrologue = 0, vmLoop = 0, lgkmLoop = -1;
  int64_t loaderWaves = 0; // load-only waves beside the wave grid's
};
InstanceSchedule instanceSchedule(const InstanceKey &k);

// The compiler's register and scratch report for the build an instance key
// binds (the build step reads hipcc's kernel-resource-usage remarks into the
// table; csrc/tools/resource_table.py): VGPRs, AGPRs and SGPRs per wave and
// scratch bytes per lane. `partialK`: the problem's K is not a multiple of
// block_k, which the hand-scheduled 16x16x32 instance serves with the
// 16x16x32 loop's build of its tile (every other instance has one build for
// all K). `known` is false for a key with no compiled kernel.
struct InstanceResources {
  bool known = false;
  int64_t vgprs = 0, agprs = 0, sgprs = 0, scratchBytes = 0;
  std::string kernel; // the kernel function the numbers come from
};
InstanceResources instanceResources(const InstanceKey &k, bool partialK = false);
// The refusal of an instance that spills ("" when it does not): the plan
// binds only instances whose registers hold the whole wave tile.
std::string spillRefusal(const InstanceKey &k, bool partialK = false);

// A 16x16x32 instance exists for this block, wave grid and stage count (in
// every output mode, plain and fused): the hand-scheduled 256x256x64 tile
// or a tile of TBK_M16_SHAPES.
bool hasMfma16Tile(int64_t bm, int64_t bn, int64_t bk, int64_t wgm, int64_t wgn,
                   int64_t stages);

// (wave grid, stages) pairs compiled for a block shape on 32x32x16 MFMA.
std::vector<std::pair<std::pair<int64_t, int64_t>, int64_t>>
compiledWaveGrids(int64_t bm, int64_t bn, int64_t bk);

} // namespace tb
