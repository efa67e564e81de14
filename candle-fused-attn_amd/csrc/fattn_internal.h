// Internal interface between the C-ABI layer (fattn_api.cpp) and the gfx950 kernels
// (fattn_kernels.hip), both compiled by hipcc. The scheduling functions below are __host__
// __device__: the kernels and the host's grid sizes use the same code.
#ifndef FATTN_INTERNAL_H
#define FATTN_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fattn {

// head_dim of the reference's kernels; the kernels here are built for 32, 64 and 128.
constexpr int kHeadDim = 64;
bool head_dim_supported(int64_t d);

// Backward tiling: a workgroup owns kBwdKeys keys of one (batch, head) and walks query tiles of
// kBwdQueryTile; per query tile one dQ partial slot per key block (split) or one dQ turn counter
// (turns).
constexpr int kBwdKeys = 64;
#ifndef BWD_QT
#define BWD_QT 16
#endif
constexpr int kBwdQueryTile = BWD_QT;

// A [b, h, s, d] operand on the device: its first element and its (batch, head, seq) strides
// in floats, head_dim contiguous.
struct View {
  const float* p;
  int64_t sb, sh, ss;
};

// Workspace of the backward, in this order, each part 256-byte aligned:
//   ctrl   64 i32                           [0] key-block ticket, [32] guard word (first, so
//                                           that its place does not depend on the shape)
//   D      [b, h, s] f32                    rowsum(dO o O)
//   turn   [b, h, ntile] i32                dQ turn counter per query tile (turn hand-over)
//   part   [nkb, b, h, ntile, kQT * d] f32 dQ partial per key block and query tile (split only)
//   arrive [b, h, nkb] u64                  per key block: the epoch of the launch that finished
//                                           it, or'ed with its XCD (split)
//   done   [b, h, ntile] u64                the epoch of the launch whose step 2 summed the tile
//   epoch  u64 (256 bytes)                  the epoch of the last step 2 launch on the workspace
// with ntile = ceil(s / kBwdQueryTile), nkb = ceil(s / kBwdKeys). `bytes_min` covers ctrl, D and
// turn (the turn hand-over), `bytes_split` all seven.
struct Workspace {
  size_t d_off, turn_off, ctrl_off, part_off, arrive_off, done_off, epoch_off, bytes_min,
      bytes_split;
};
Workspace workspace_layout(int64_t b, int64_t h, int64_t s, int64_t d);
constexpr int kCtrlTicket = 0;
constexpr int kCtrlGuard = 32;
// dQ sums inside step 2 (split mode): a query tile is summed in step 2 once every key block it
// needs has finished, from partials stored and read at device scope (so whatever XCDs the key
// blocks ran on); step 3, where it runs, sums what step 2 left. Non-causal, workgroups appended to
// step 2's grid do the sums; causal, each key block's own workgroup sums, after its walk, the
// tiles whose last contributor it is. Every step 2 launch carries its own epoch (a 64-bit value
// unique to the launch, low 3 bits zero): the key blocks' arrivals and the done flags hold it, so
// nothing needs clearing between launches and no stale or uninitialised value passes for a
// current one (but with a 2^-64 chance). The summing workgroups poll at most kSumMaxBlocks
// arrival slots.
constexpr int kSumMaxBlocks = 256;
constexpr int kSumTiles = 3;  // query tiles per summing workgroup
// Causal: the query tiles whose last contributor is key block kb of `keys` keys (its diagonal
// tiles; keys / kBwdQueryTile of them, fewer at the end of the sequence).
__host__ __device__ inline void own_tiles(int kb, int keys, int ntile, int* j0, int* j1) {
  const int n = keys / kBwdQueryTile;
  *j0 = kb * n;
  *j1 = *j0 + n < ntile ? *j0 + n : ntile;
}

// Workgroups are dealt to the 8 XCDs round-robin (workgroup id % 8). xcd_remap gives each XCD a
// contiguous range of logical items, so logical neighbours (the key blocks of one (b, h)) share
// one L2: workgroup id runs item (id % 8) F + id / 8 with F = (total rounded down to a multiple
// of 8) / 8; the last total % 8 items run as themselves.
__host__ __device__ inline int xcd_remap(int id, int total) {
  const int full = total & ~7;
  if (id >= full) return id;
  return (id & 7) * (full >> 3) + (id >> 3);
}
// The XCD that runs logical item `item` of xcd_remap (its inverse, taken mod 8).
__host__ __device__ inline int item_xcd(int item, int total) {
  const int full = total & ~7;
  return item >= full ? (item & 7) : item / (full >> 3);
}

// The dQ sums in step 2 (split). Non-causal: workgroups appended to step 2's grid; workgroup
// n_main + 8 m + x runs on XCD x (workgroups go to the XCDs round robin on MI355X). xcd_remap
// gives XCD x the (b, h)-major key blocks [x F, (x + 1) F), F = floor(nkb b h / 8), and deals the
// rest (fewer than 8) round robin. Summing workgroup m < mc nchunk of XCD x takes chunk
// m % nchunk of the (m / nchunk)-th (b, h) whose last key block is among XCD x's, so that the
// sums dispatched first wait for the key blocks dispatched first; the workgroups after those take,
// in (b, h) order, the (b, h)s whose last key block is among the rest. Causal: every key block
// sums the tiles it completes. The partials are read at device scope, so the XCDs order the waits
// but are not needed for correctness. on = 0: no sums (step 3 sums every tile).
struct SumPlan {
  int on;
  int nchunk;  // chunks of kSumTiles query tiles per (b, h)
  int nkb;     // key blocks per (b, h)
  int mc;      // (non-causal) the most (b, h)s one XCD's range holds
};
// The (b, h)s whose last key block lies in XCD x's range of key blocks: lo .. hi (empty if
// hi < lo); consecutive over x, from 0 to 8 F / nkb - 1.
__host__ __device__ inline int sum_range_lo(int x, int F, int nkb) {
  return (x * F + nkb) / nkb - 1;  // ceil((x F + 1) / nkb) - 1
}
__host__ __device__ inline int sum_range_hi(int x, int F, int nkb) { return (x + 1) * F / nkb - 1; }
__host__ __device__ inline SumPlan sum_plan(int BH, int nkb, int ntile, int d, int causal) {
  SumPlan p{0, (ntile + kSumTiles - 1) / kSumTiles, nkb, 0};
  if (nkb > kSumMaxBlocks || BH <= 0) return p;
  p.on = 1;
  if (!causal) {
    const int F = nkb * BH / 8;
    for (int x = 0; x < 8; ++x) {
      const int n = sum_range_hi(x, F, nkb) - sum_range_lo(x, F, nkb) + 1;
      p.mc = n > p.mc ? n : p.mc;
    }
  }
  return p;
}
// Workgroups appended to step 2's grid for the non-causal sums (a multiple of 8).
__host__ __device__ inline int sum_blocks(SumPlan p, int BH, int causal) {
  if (causal || !p.on) return 0;
  const int left = BH - 8 * (p.nkb * BH / 8) / p.nkb;
  return 8 * p.mc * p.nchunk + (left * p.nchunk + 7) / 8 * 8;
}
// Non-causal summing workgroup m of XCD x (workgroup n_main + 8 m + x): the (b, h) it sums and
// its first query tile. False for a workgroup with nothing to sum (past the plan or past b h),
// and always when causal (no summing workgroups).
__host__ __device__ inline bool sum_target(SumPlan p, int x, int m, int BH, int causal, int* bh,
                                           int* j0) {
  if (causal || !p.on) return false;
  const int F = p.nkb * BH / 8;
  if (m < p.mc * p.nchunk) {
    const int b0 = sum_range_lo(x, F, p.nkb) + m / p.nchunk;
    if (b0 > sum_range_hi(x, F, p.nkb) || b0 >= BH) return false;
    *bh = b0;
    *j0 = m % p.nchunk * kSumTiles;
    return true;
  }
  const int idx = (m - p.mc * p.nchunk) * 8 + x, left0 = 8 * F / p.nkb;
  if (idx >= (BH - left0) * p.nchunk) return false;
  *bh = left0 + idx / p.nchunk;
  *j0 = idx % p.nchunk * kSumTiles;
  return *bh < BH;
}
// Keys per key block of the split step 2 (d <= 64): kBwdKeys, or twice that (each wave owning two
// groups of 16 keys) for long non-causal sequences at d 64. The sums' plan, step 3 and the
// workspace's slots (sized for kBwdKeys) follow it.
int bwd_split_keys(int64_t b, int64_t h, int64_t s, int d, int causal);
// Whether step 2 sums dQ tiles for this shape (the plan has (b, h)s to sum and the sums are on).
bool bwd_step2_sums(int64_t b, int64_t h, int64_t s, int d, int causal);
// Workgroups appended to step 2's grid for the non-causal sums (0 when causal or without sums).
int64_t bwd_sum_blocks(int64_t b, int64_t h, int64_t s, int d, int causal);
// Test hooks (the C ABI lets a process use them only when it opted in at load). Step 2's sums on
// (the default) or off for every later backward of the process, so that a test can compare both;
// returns the previous setting.
bool set_step2_sums(bool on);
// The non-causal summing workgroups of XCD x sum the (b, h)s of XCD x + shift (mod 8) in every
// later launch, so that their partials come from another XCD; returns the previous shift.
int set_sum_shift(int shift);
// Step 2's dQ sums of (b, h) pair `bh` (of the whole backward; -1: none, the default) give up
// before their first poll in every later launch, as a wait that timed out would; returns the
// previous pair.
int set_give_up_bh(int bh);
// The three hooks' current settings: step 2's sums on, the sum shift, the give-up pair.
void test_hook_state(int64_t out[3]);
// Step 3's grid: one workgroup per query tile, or (with step 2's sums) at most 256 workgroups
// that each check a range of tiles and sum those not done.
int64_t bwd_dq_grid(int64_t b, int64_t h, int64_t s, int d, int causal);

// Launchers (fattn_kernels.hip). They assume validated arguments; they return a hipError_t
// value as int (0 = launched).
int launch_forward(View q, View k, View v, float* o, float* lse, int b, int h, int s, int d,
                   float scale, int causal, void* stream);
int launch_bwd_prep(const float* o, View d_o, float* dsum, int* turn, int* ctrl, int b, int h,
                    int s, int d, void* stream);
// part == nullptr: the turn hand-over (dQ final after step 2; D from step 1); else the split
// partials, which step 3 (launch_bwd_dq) sums into dQ (D computed from o here, no step 1).
// arrive / done / epoch_slot (split, d <= 64): step 2's dQ sums, tagged with `epoch`.
// bh0, nbh (split, d <= 64): the (b, h) pairs bh0 .. bh0 + nbh - 1 only, whose partials, slots
// and flags sit in a workspace laid out for nbh pairs (workspace_layout(1, nbh, s, d)); otherwise
// 0 and b h.
int launch_bwd_main(View q, View k, View v, View d_o, const float* o, const float* lse,
                    const float* dsum, float* dqkv, float* part, unsigned long long* arrive,
                    unsigned long long* done, unsigned long long* epoch_slot,
                    unsigned long long epoch, int* turn, int* ctrl, int b, int h, int s, int d,
                    float scale, int causal, int bh0, int nbh, int sums_final, void* stream);
// Whether step 2's sums cover every query tile of a launch over nbh of the b h pairs (then no
// step 3 need follow it).
bool bwd_step2_sums_all(int64_t nbh, int64_t b, int64_t h, int64_t s, int d, int causal);
// Step 3: dQ of every query tile that step 2 did not sum (done: null, none did); then the done
// flags and arrival slots are zeroed. bh0, nbh: as step 2's.
int launch_bwd_dq(const float* part, unsigned long long* done, unsigned long long* arrive,
                  const unsigned long long* epoch_slot, float* dqkv, int b, int h, int s, int d,
                  float scale, int causal, int bh0, int nbh, void* stream);

// The device address of the library's static scratch (FATTN_STATIC_SCRATCH_BYTES, the workspace
// of fattn_bwd_f32_noalloc) on the device that runs `stream`; a hipError_t value as int.
int static_scratch(void* stream, void** out);

// Grid sizes the launchers will use (for range checks before launching).
int64_t forward_blocks(int64_t b, int64_t h, int64_t s, int causal, int d);
int64_t bwd_main_blocks(int64_t b, int64_t h, int64_t s);
int64_t bwd_prep_blocks(int64_t b, int64_t h, int64_t s, int d);
int64_t bwd_dq_blocks(int64_t b, int64_t h, int64_t s);
// Whether step 1 (D, counters) must run: the turn mode, and the split mode at d 128 past
// kOwnDMaxBlocks key blocks per (b, h) (fewer: its step 2 forms D itself).
bool bwd_needs_prep(bool split, int d, int64_t s);
// D 128, split: step 2 forms D = rowsum(dO o O) itself (few key blocks per (b, h)).
bool bwd_own_d(int64_t s, int d);

}  // namespace fattn

#endif  // FATTN_INTERNAL_H
