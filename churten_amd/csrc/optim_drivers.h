// optim_drivers.h -- the gfx950 kernels of the fused optimizer step and their
// launchers.
//
// Structure. Each optimizer is a policy (AdamPolicy, SgdPolicy, AdagradPolicy,
// AdagradF32Policy): its per-replica prologue (hyperparameters, bias
// corrections, is_first_step, corrected_lr) and its per-element update, both
// from optim_math.h, over a parameter type T and an optimizer-state type S
// (S = T, or bfloat16 state next to float32 parameters). Four drivers move the
// bytes, identically for every policy:
//
//   stream_kernel   unit inner stride (the consolidated layout `State`
//                   produces, and ragged or misaligned rows): one wavefront
//                   per tile (1-4 packs of 4 or 8 elements per thread by
//                   operand types), non-temporal 16-byte loads and stores,
//                   tiles on the row's boundaries of the tile size (tiles
//                   never share a cache line) and one head tile per row for
//                   what lies before the first, the few elements off the
//                   pack grid one at a time;
//                   large launches cap residency per CU. Operands at another
//                   16-byte phase than the parameters take element-aligned
//                   packs (the ANY variant).
//   column_kernel   unit replica stride on every operand (transposed views,
//                   as an outer vmap over a non-leading dimension gives): each
//                   thread keeps one replica and walks columns, so the threads
//                   of a workgroup read consecutive replicas -- contiguous
//                   memory. Non-temporal where workgroups own their cache
//                   lines and a wavefront has no frozen replica; the replica
//                   blocks of a column block share an XCD when there are
//                   several.
//   element_kernel  any other inner strides: one element per access.
//   segment_kernel  the gradient arrives as one tensor per parameter (a segment
//                   table) instead of the consolidated (R, T) gradient buffer:
//                   the gradient scatter of the training step is fused into the
//                   update. Optionally the consolidated gradient is written on
//                   the way through, so `flat_grads` stays what it would have
//                   been. Same access pattern as stream_kernel over each
//                   segment's columns, whatever the segment's offset.
//
// Operands are ordered [0] param, [1] grad (both T), [2..] optimizer state (S;
// Adam: exp_avg, exp_avg_sq, [max_exp_avg_sq]; SGD: [momentum_buffer];
// Adagrad: state_sum). The dense drivers never write the grad; the segmented
// driver may store the gradient it read into the consolidated buffer.
//
// Work decomposition. Rows are cut into tiles of consecutive elements
// (segments into tiles of their own); a 1-D grid enumerates (replica, tile)
// pairs replica-major, so blockIdx.x gives both and no grid dimension caps R.
// A workgroup first reads its replica's active flag: a frozen replica is a
// workgroup-uniform early exit, so its rows are never read or written (they stay
// bit-identical, and a replica frozen at step 0 never evaluates 1 - beta^0 = 0).
// Active workgroups read the replica's hyperparameters once (uniform address:
// scalar loads) and read the per-replica constants from the call's workspace
// or derive them (float32 Adam: once per wavefront, the work spread over its
// lanes), then stream their tile.
// All drivers inline the same per-element update, so the same element gives
// the same bits whichever driver processed it.
//
// (column_kernel instead enumerates (column block, replica block) pairs, in
// an XCD-aware order when a column has several replica blocks, and tests the
// flag per thread.)
//
// Everything is enqueued on the caller's stream; nothing is allocated.

// This header holds the policies, the drivers and their host-side launchers;
// optim_dispatch.h dispatches the C ABI of include/churten_optim.h onto them.
// Everything is in an anonymous namespace: a translation unit that includes it
// gets its own kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <initializer_list>
#include <type_traits>

#include "../../include/churten_optim.h"
#include "optim_math.h"

namespace churten {
namespace {

// Launch shape, measured on the MI355X over the 52 GB north-star state:
// non-temporal vector loads and stores of 4-element packs (non-temporal hints
// on both loads and stores were worth ~10% over plain accesses, either alone
// nothing). The streaming driver runs one wavefront per workgroup under a
// residency cap (each policy's shape below): of 64/128/256 threads x 1/2/4
// packs x 8-24 resident waves per CU, that was fastest, ahead of 128 x 2 with
// its best cap by 2-6% and uncapped 128 x 2 by 6-10%. The segmented driver
// and the scatter mostly run one wavefront too; the element and column
// drivers and a few segmented forms keep 128 or 256 threads, where their own
// sweeps put them. kThreads / kPer are the defaults those start from.
constexpr int kThreads = 128;
constexpr int kPack = 4;
constexpr int kUnroll = 2;
constexpr int kPer = kPack * kUnroll;  // elements per thread per tile
constexpr int kStreamThreads = 64;

// Tile boundaries sit on 256-byte boundaries of the (R, T) rows (the
// streaming driver's on boundaries of its own tile size, a multiple of 256
// bytes). Consecutive tiles run on different XCDs (each with its own L2); a
// 128-byte line split between two of them is fetched twice and written back
// as two partial lines. Measured on the MI355X with the same buffers viewed
// 16 / 64 / 128 / 0 bytes off a 256-byte boundary: the Adam step took
// 19% / 8% / 1% / 0% longer.
constexpr uint32_t kAlignBytes = 256;
template <typename T>
constexpr uint32_t align_elems() {
  return kAlignBytes / sizeof(T);
}

// Rows' phases (res0 / rmod) are kept modulo this many bytes: a multiple of
// every alignment the drivers use (256 bytes for the segmented and scatter
// walks, the streaming driver's tile size: 1-8 KB). All are powers of two, so
// a phase product res0 + r * rmod that wraps in 32 bits keeps its residue.
constexpr uint32_t kPhaseBytes = 16384;
template <typename T>
constexpr uint32_t phase_elems() {
  return kPhaseBytes / sizeof(T);
}

// N consecutive elements of one operand: 4 in the drivers' usual pack (16 B
// for float32, 8 B for 16-bit types, 32 B for float64); the streaming driver
// takes 8 where a policy has 16-bit operands (kStreamPack), so those move
// 16 B per access too.
template <typename T, int N = kPack>
struct alignas(sizeof(T) * N) Pack {
  T v[N];
};

// A pack as raw 32-bit words, so it can go through the non-temporal builtins.
template <typename T, int N = kPack>
using PackBits = uint32_t __attribute__((ext_vector_type(sizeof(T) * N / 4)));

// Streaming accesses: every byte of the optimizer state is touched exactly
// once per step, so the loads and stores carry the non-temporal hint (NT).
// Launches whose operands fit the 256 MB MALL several times over take plain,
// cache-allocating accesses instead (NT = false): back-to-back steps then hit
// the MALL (see the streaming driver's launch).
template <bool NT, typename V>
__device__ __forceinline__ V load_bits(const V* p) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}
template <bool NT, typename V>
__device__ __forceinline__ void store_bits(V* p, V v) {
  if constexpr (NT) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = v;
  }
}

template <bool NT = true, typename T, int N>
__device__ __forceinline__ Pack<T, N> load_stream(const Pack<T, N>* p) {
  return __builtin_bit_cast(Pack<T, N>,
                            load_bits<NT>(reinterpret_cast<const PackBits<T, N>*>(p)));
}

template <bool NT = true, typename T, int N>
__device__ __forceinline__ void store_stream(Pack<T, N>* p, const Pack<T, N>& v) {
  store_bits<NT>(reinterpret_cast<PackBits<T, N>*>(p), __builtin_bit_cast(PackBits<T, N>, v));
}

// A pack whose value the compiler cannot know, at no cost (no instruction):
// the value a pack can hold where a thread has nothing to load. Left undefined
// there, a pack lets the compiler fold the conversion of a loaded 16-bit pack
// into the branch that loads it, and the wavefront then waits for that load
// right there, before it issues the next loads or its other work.
template <typename T, int N>
__device__ __forceinline__ void opaque(Pack<T, N>& x) {
  PackBits<T, N> b;
  asm volatile("" : "=v"(b));
  x = __builtin_bit_cast(Pack<T, N>, b);
}

// Packs at addresses that are only element-aligned: operands whose 16-byte
// boundaries do not line up with the parameters' (a column view at another
// offset, a per-parameter gradient's rows). gfx950 code runs in unaligned
// access mode, and hipcc emits the same single global_load/store_dwordx4
// (dwordx2 for 16-bit types) for these types as for an aligned pack; on an
// aligned address the access is the aligned one.
template <typename T, int N = kPack>
using PackBitsU = uint32_t
    __attribute__((ext_vector_type(sizeof(T) * N / 4), aligned(sizeof(T))));

template <bool NT = true, int N = kPack, typename T>
__device__ __forceinline__ Pack<T, N> load_stream_any(const T* p) {
  return __builtin_bit_cast(Pack<T, N>,
                            load_bits<NT>(reinterpret_cast<const PackBitsU<T, N>*>(p)));
}

template <bool NT = true, int N = kPack, typename T>
__device__ __forceinline__ void store_stream_any(T* p, const Pack<T, N>& v) {
  store_bits<NT>(reinterpret_cast<PackBitsU<T, N>*>(p), __builtin_bit_cast(PackBitsU<T, N>, v));
}

// The N-element packs of an operand from a given element on: aligned to the
// pack wherever the parameters' packs are (ANY = false, the usual case: the
// compiler knows the alignment) or only element-aligned (ANY = true). Indexed
// by pack.
template <bool ANY, typename T, bool NT = true, int N = kPack>
struct Packs;

template <typename T, bool NT, int N>
struct Packs<false, T, NT, N> {
  Pack<T, N>* p = nullptr;
  Packs() = default;
  __device__ explicit Packs(T* e) : p(reinterpret_cast<Pack<T, N>*>(e)) {}
  __device__ Pack<T, N> load(int64_t i) const { return load_stream<NT>(p + i); }
  __device__ void store(int64_t i, const Pack<T, N>& v) const { store_stream<NT>(p + i, v); }
};

template <typename T, bool NT, int N>
struct Packs<true, T, NT, N> {
  T* p = nullptr;
  Packs() = default;
  __device__ explicit Packs(T* e) : p(e) {}
  __device__ Pack<T, N> load(int64_t i) const { return load_stream_any<NT, N>(p + i * N); }
  __device__ void store(int64_t i, const Pack<T, N>& v) const {
    store_stream_any<NT, N>(p + i * N, v);
  }
};

constexpr int kMaxOperands = 5;

// (R, T) operands. `data[i]` is element (0, 0) of operand i.
template <typename T>
struct Operands {
  T* data[kMaxOperands];
  int64_t stride_r[kMaxOperands];
  int64_t stride_t[kMaxOperands];
};

// (R,) inputs: the step counter, up to five hyperparameter vectors and the mask.
// `pre`: the call's per-replica constants (kPreWords doubles per replica,
// replica r at pre + kPreStride * r), written by the preparation launch; null
// when the workgroups derive them themselves.
// `ilp_rows`: which rows torch's fused kernels would run on their vector path
// (see ilp_row).
template <typename T>
struct Vectors {
  const T* steps;
  const T* h[5];
  const uint8_t* mask;
  const double* pre;
  uint32_t ilp_rows;
};

// Whether row r takes the vector path of torch's fused optimizer kernels (and
// of the reference's row kernel, adagrad.cu:119-133): the row's length a
// multiple of 4 and every operand's row pointer aligned to 4 elements, with
// unit inner stride (ATen MultiTensorApply's kILP = 4; its chunks start at
// multiples of 4). `rule` is 0 when no row does; else bit 0 is set and
// operand b < 3 adds its base's element offset modulo 4 (bits 1+4b, 2+4b) and
// its row stride modulo 4 (bits 3+4b, 4+4b); row r is aligned in operand b
// when their (offset + r * stride) is 0 modulo 4.
__device__ __forceinline__ bool ilp_row(uint32_t rule, uint32_t r) {
  if (rule == 0) return false;
  bool ok = true;
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    const uint32_t res = (rule >> (1 + 4 * b)) & 3u;
    const uint32_t mod = (rule >> (3 + 4 * b)) & 3u;
    ok = ok && ((res + r * mod) & 3u) == 0;
  }
  return ok;
}

// Doubles per replica in a workspace of per-replica constants.
constexpr int kPreStride = 2;

// Tiles of a driver's tile size per row. res0 is the parameter base's element
// offset and rmod its row stride, both modulo kPhaseBytes in elements of the
// parameter type. For the streaming driver, row r's first boundary of the tile
// size (TILE elements) lies head(r) = (TILE - (res0 + r * rmod) % TILE) % TILE
// elements in; its tiles k >= 1 start there, and its tile 0 takes the head
// (packs from the first pack boundary, fewer than a pack before it one element
// at a time) and the row's fewer than a pack of tail elements. Where every
// operand shares the parameter's phase modulo the pack, the packs are aligned
// in all of them (else the ANY variants run).
struct Grid {
  int64_t T;
  uint32_t tiles_per_row;
  uint32_t res0, rmod;
  // Workgroups at the start of the grid that take each row's tile 0 (the
  // streaming driver's head tiles: one per row), before the rows' other tiles.
  uint32_t heads;
  // Division by tiles_per_row as a multiply and shifts (div_tiles).
  uint32_t magic, sh1, sh2;
};

// q = m / d for every 32-bit m, with d = tiles_per_row fixed per launch: the
// round-up method of Granlund and Montgomery ("Division by invariant integers
// using multiplication", PLDI 1994, fig. 4.1). With l = ceil(log2 d),
// magic = floor(2^32 (2^l - d) / d) + 1, t = mulhi(m, magic) and
// q = (t + ((m - t) >> min(l, 1))) >> max(l - 1, 0). Five scalar instructions
// where the generic 32-bit divide takes about 25, several of them vector and
// one a reciprocal; it is on the path from a workgroup's start to its first
// load (config 2 +1.0%, config 5 +0.2% in a same-process A/B). set_div_tiles
// computes the constants on the host.
__device__ __forceinline__ uint32_t div_tiles(const Grid& g, uint32_t m) {
  const uint32_t t = __umulhi(m, g.magic);
  return (t + ((m - t) >> g.sh1)) >> g.sh2;
}
inline void set_div_tiles(Grid& g) {
  const uint32_t d = g.tiles_per_row;
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  g.magic = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  g.sh1 = l < 1 ? l : 1;
  g.sh2 = l > 1 ? l - 1 : 0;
}

// Integer minimum for tile bounds (a plain compare-and-select; HIP's generic
// min template goes through double for 64-bit integers).
__device__ __forceinline__ int64_t imin(int64_t a, int64_t b) { return a < b ? a : b; }

template <int64_t TILE>
__device__ __forceinline__ void tile_of_block(const Grid& g, uint32_t& r,
                                              int64_t& t0) {
  const uint32_t tile = blockIdx.x;
  r = tile / g.tiles_per_row;
  t0 = int64_t(tile - r * g.tiles_per_row) * TILE;
}

// The streaming driver's grid: workgroup b < heads takes row b's tile 0;
// the others take row r's tile k + 1 (t0 = (k + 1) * TILE) in row-major order,
// the same order as a grid without head tiles, shifted by `heads`.
template <int64_t TILE>
__device__ __forceinline__ void stream_tile_of_block(const Grid& g, uint32_t& r,
                                                     int64_t& t0) {
  const uint32_t b = blockIdx.x;
  if (b < g.heads) {
    r = b;
    t0 = 0;
    return;
  }
  const uint32_t m = b - g.heads;
  r = div_tiles(g, m);
  t0 = int64_t(m - r * g.tiles_per_row + 1) * TILE;
}

template <typename T>
__device__ __forceinline__ double hyper_at(const T* h, uint32_t r) {
  return static_cast<double>(widen(h[r]));
}

// Lane `lane`'s x, for every lane of the wavefront (that lane must be active).
__device__ __forceinline__ double wave_lane(double x, int lane) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(b), lane);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(b >> 32), lane);
  return __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo);
}

// ---------------------------------------------------------------------------
// Policies
// ---------------------------------------------------------------------------
// Residency cap of the streaming driver. A large streaming launch runs faster
// with fewer one-wave workgroups resident per CU than the register budget
// allows (24): measured on the MI355X over config-5-sized fp32 state (same
// buffers, interleaved, several processes), with every workgroup deriving its
// replica's constants: 14 per CU for Adam, 12 with amsgrad and 16 for
// Adagrad, +3-10% over no cap; bfloat16 state lost with any cap and fp64
// gained nothing. With the constants precomputed the caps move (below, next to
// the policies). The cap is dynamic LDS that the kernel never touches (the
// smallest 256-byte multiple that fits only n workgroups in the CU's 160 KiB),
// so it changes residency and nothing else. `kStreamLds` / `kStreamLdsPre` are
// each policy's reservations; small launches (under kCapMinElems elements of
// the (R, T) operands, 8192 tiles of 512) launch without them, since there the
// cap would only serialise the launch (config 1 lost 16% with one). The
// segmented driver runs uncapped (its shapes are next to segment_tile).
constexpr uint32_t kLdsPerCU = 160 * 1024;
constexpr uint32_t lds_for_residency(uint32_t n) {
  uint32_t x = (kLdsPerCU / n) / 256 * 256;
  while (kLdsPerCU / x > n) x += 256;
  return x;
}
template <typename T, typename S>
constexpr bool kFp32State = std::is_same<T, float>::value && std::is_same<S, float>::value;
template <typename T, typename S>
constexpr uint32_t residency_lds(uint32_t n) {
  return kFp32State<T, S> ? lds_for_residency(n) : 0u;
}
template <typename T, typename S>
constexpr bool kBf16State = std::is_same<T, float>::value && std::is_same<S, bf16_t>::value;
template <typename T, typename S>
constexpr bool kHalfAll = std::is_same<T, _Float16>::value && std::is_same<S, _Float16>::value;
constexpr int64_t kCapMinElems = int64_t(8192) * 512;

// Launches whose (R, T) operands take at most this many bytes run the SMALL
// streaming shape (plain accesses, the policy's kStreamUnrollSmall, no cap):
// the MI355X's 256 MB MALL then keeps them between back-to-back steps.
// Measured on configs 1-4 (prep + update through the C ABI, 200 launches, 5
// rounds): config 1 (34 MB of Adam operands) 11.7 us plain with 2 packs
// against 13.0 non-temporal; config 3 (209 MB, SGD) 32.0 us plain with 1 pack
// (2 / 4 / 8 packs: 33.9 / 32.6 / 32.2) against 35.8; configs 2 and 4 (531 /
// 419 MB) lose 11-16% with plain accesses, so they stay non-temporal.
constexpr int64_t kMallBytes = int64_t(256) << 20;

// Launches above the MALL with at most kMidBytes of (R, T) operands reserve
// each policy's kStreamLdsMid instead of its large-launch cap (with a
// workspace). Measured with a launch-shape sweep at config 2's size (100 x 265,484,
// 75% active; three runs on two boxes): float32 Adam at cap 20 5.85-5.94 TB/s
// against 5.66-5.74 at its cap of 14, and with amsgrad 5.83-5.91 against
// 5.73-5.79 at its cap of 12. From 2 GB of operands on (R = 128, T = 1M to
// 8M) the large-launch caps were best or within 0.3%. (With the active flag
// read through the scalar cache the mid-size caps moved to 14, 12 with
// amsgrad; see the policies.)
constexpr int64_t kMidBytes = int64_t(1) << 30;

// Packs per thread of the streaming driver, by operand types: float32
// throughout, float32 params with bfloat16 state, 16-bit params, float64.
// Measured per policy on config-5-sized state (1/2/4/8 packs, one process per
// sweep, two sweeps): float32 keeps 2 (under its residency cap; 1 with
// precomputed constants, below); bfloat16 state wants 4 for Adam (+13%; 2 with
// precomputed constants, below) but 1 for SGD and Adagrad (+8-15%); float64 is
// flat. 16-bit params and state take one 8-element (16-byte) pack per thread,
// uncapped, for large launches (Adagrad with precomputed constants: 4, below).
// Against the previous 4-element packs x 8 (config-5 buffers, half and
// bfloat16 timed on the same storage, 5-6 interleaved rounds, three sweeps on
// different boxes): Adam +4-8% (one box: half -2%), SGD +7-9%, float32-math
// Adagrad +10-12%, Adagrad -1% to +0.2%; two and four packs per thread and
// caps of 10-20 were slower on average. Small launches keep 2048-element tiles
// (four 8-element packs).
// kLateStores (per policy): the streaming driver stores a thread's packs
// after all of its arithmetic instead of each pack right after its own.
// Measured interleaved on the config-5 buffers: Adam +0.6-0.9% (three boxes),
// Adam with bfloat16 moments +1.9-2.0%, SGD +0.2-0.3%, Adagrad -1.2%; Adam
// with amsgrad -2.2% (config 2 scaled to 1200 replicas; -0.8% at config 2)
// against +2.8% for Adam at config 1; float64 Adam -31% (5.06 -> 3.47 TB/s),
// float16 Adam -2%, bfloat16-parameter Adam +1.4%. So only float32 parameters
// (with float32 or bfloat16 state) of Adam without amsgrad and of SGD store
// late. The segmented driver keeps per-pack stores for every policy: late
// ones lost 0.6-0.8% there.
// Elements per pack of the streaming driver: 16 B per lane and access, so a
// wavefront's access covers 1 KB of consecutive bytes. 8 where parameters and
// state are 16-bit, 2 for float64, else 4. With float32 parameters next to
// bfloat16 state a pack stays 4 elements (8 B of state): 8-element packs there
// make the float32 operands' accesses 32 B apart per lane, measured 5-15%
// slower on the config-5 buffers. float64 had 4-element packs (32 B apart per
// lane, two accesses each covering every other 16 B of 2 KB); 2-element packs
// with the same packs per thread, same-process A/B on 64 x 4M doubles, 4
// rounds: Adam +23% with a workspace (6.53 TB/s) and +13% without, SGD with
// momentum +17%, Adagrad +17%, config 1's shape in float64 +5%.
template <typename T, typename S>
constexpr int stream_pack() {
  return sizeof(T) == 2 && sizeof(S) == 2 ? 8 : std::is_same<T, double>::value ? 2 : kPack;
}

template <typename T, typename S>
constexpr int stream_unroll(int fp32, int bf16_state, int narrow, int wide) {
  return std::is_same<T, double>::value ? wide
         : sizeof(T) == 2              ? narrow
         : !std::is_same<S, T>::value  ? bf16_state
                                       : fp32;
}

// Every policy has a parameter/gradient type T and an optimizer-state type S:
// S == T is the reference's contract; S = bf16_t with T = float keeps the
// moments (momentum buffers, sums) in bfloat16 while the element math and the
// parameters stay in float32 (the state is widened on load and rounded to
// nearest-even on store).
//
// Per-replica constants. `prologue<false>` derives a replica's constants in
// every workgroup (Adam: two fp64 pow and the step size's divide; Adagrad: an
// fp64 divide); `prologue<true>` reads them from the call's workspace, where
// the preparation launch (`precompute`, once per replica and call, after the
// step bump) put them. Both give the same bits: the workspace holds the
// math-type values widened to double (Adam's divisor of sqrt(v) is a double
// already). kPreWords is the number of such doubles (0: nothing worth
// hoisting, the policy never reads a workspace). `reads_state` is decided from
// the (R,) vectors alone, so the drivers issue their loads before the prologue.
// `decays` / `drop_decay`: whether the replica's weight-decay term is live, and
// a copy of its constants with the decay set to a literal zero (the element
// math then skips the term, exactly as it does for a zero decay at run time).
// `kVariant` / `variant` / `set_variant`: a per-replica choice between two
// forms of the element math (float16 Adagrad's once- or twice-rounded state
// sum), which the streaming and segmented drivers branch on once per
// workgroup with the choice set to a literal (with_variant).
//
// Streaming shape with a workspace (kStreamUnrollPre, kStreamLdsPre). Without
// the pow in every workgroup, float32 Adam runs fastest with one pack per
// thread (256-element tiles) under the same cap of 14 workgroups per CU:
// 6.51 against 6.15 TB/s for the per-workgroup form (two boxes, config-5
// buffers, interleaved); two packs with precomputed constants reached 6.22
// at that cap and 6.36 at 8, and a workgroup walking 2-8 consecutive tiles
// with one prologue 6.10-6.22. The same sweep per policy (config-5 shape,
// 3 interleaved rounds, two boxes; one pack against the old two):
//   Adam with amsgrad    1 pack, cap 12: 6.34-6.36 TB/s (2 packs: 5.85)
//   Adagrad (fp64 math)  1 pack, cap 20: 6.45-6.49 (2 packs, cap 16: 5.70;
//                        caps 18-24 within 0.7% of each other)
//   Adagrad, fp32 math   1 pack, cap 20: 6.52 (2 packs, cap 16: 5.84)
// SGD has no workspace, but with its loads issued before the prologue its
// buffered float32 form also runs one pack per thread, cap 20: 6.46-6.60
// against 6.13 for two packs at cap 14. bfloat16-state SGD and Adagrad (1
// pack, uncapped) and float64 (2 packs) kept their shapes: nothing else in the
// sweep beat them. 16-bit parameters: one 8-element pack, uncapped (above).
// Rechecked after Adam's divide by bias_correction2_sqrt became a multiply
// (packs 1/2/4 x caps 10-20 and uncapped, 3 interleaved rounds per box, up to
// three boxes): float32 Adam, Adam with amsgrad, SGD and both Adagrads keep
// their shapes; two changes:
//   Adam, bf16 moments   2 packs, cap 12: 6.21-6.26 TB/s (4 packs, cap 12:
//                        6.00-6.02; 1 pack, cap 20: 6.21-6.22)
//   Adagrad, 16-bit      4 packs of 8, uncapped: half 6.14-6.18, bfloat16 6.07
//   parameters           (1 pack: half 5.65-5.88, bfloat16 5.75)
// Adam and SGD with 16-bit parameters stayed within 2% of one pack, uncapped.
// Rechecked once more after the zero-aware square root (up to three boxes,
// each shape in 2-3 processes): float16 Adam moved to one pack under a cap
// of 20 and bfloat16 SGD to two packs under a cap of 20 (at the policies);
// float16 SGD and 16-bit Adagrad kept their shapes.
// Retuned with the active flag read through the scalar cache (kScalarMask):
// a workgroup then issues its loads sooner, and the best caps moved down.
// Sweep per policy (packs 1/2/4 x caps 8-24 and uncapped, both flag reads,
// config-5 buffers unless noted, 3 interleaved rounds, mean GB/s; old shape
// with the vector read -> new):
//   Adam                   1 pack, cap 14 -> cap 12: 6432 -> 6601
//   Adam, mid size         1 pack, cap 20 -> cap 14 (config-2 rows without
//                          amsgrad): 5876 -> 6118
//   Adam + amsgrad, mid    1 pack, cap 20 -> cap 12 (config 2): 5905 -> 6054
//   Adam, no workspace     2 packs, cap 14 -> cap 10: 6266 -> 6340
//   Adam, bf16 moments     2 packs, cap 12 -> 1 pack, cap 16: 6184 -> 6462
//   Adam, 16-bit params,   1 pack, uncapped -> 4 packs: half 4559 -> 6258,
//   no workspace           bfloat16 4555 -> 6097
//   Adam, bf16 params      1 pack, uncapped -> cap 16: 6136 -> 6237
//   Adam, half params      1 pack, cap 20 (kept): 6181 -> 6248
//   Adagrad                1 pack, cap 20 -> cap 14: 6445 -> 6605 (config 4,
//                          mid size, cap 24 -> 14: 6587)
//   Adagrad, no workspace  2 packs, cap 16 -> 1 pack: 6347 (cap 14) -> 6524
//   Adagrad, bf16 state    1 pack, uncapped -> cap 20: 6331 -> 6531
//   SGD with momentum      1 pack, cap 20 (kept): 6518 -> 6608
// Adam with amsgrad (large launches) and bfloat16-state SGD stayed within
// 0.5% either way and kept their shapes. 16-bit SGD and Adagrad ran slower
// with the scalar read (bfloat16 SGD -5% at its shape) and keep the vector
// read; float64 kept it too until swept on its own (float64 Adam, SGD with
// momentum and Adagrad now read it scalar, at the policies). Same-process
// A/B of the whole change against the previous build (6 rounds): config 5
// +2.7%, config 2 +2.1%, config 3 +1.3% (SGD's MALL-resident launches read
// it scalar too), config 4 +0.4%, bfloat16 moments +5.1%, Adagrad on the
// config-5 buffers +2.3%, half / bfloat16 params +2.6% / +0.6%; config 1 is
// unchanged (Adam's MALL-resident launches keep the vector read: -1.3% with
// the scalar one).

// Without a workspace, float32 Adam derives its constants once per wavefront
// (wave_prologue: the two pow and two divides spread over even and odd lanes,
// 280 VALU instructions per workgroup instead of 425), and with it amsgrad
// moved to one pack per thread. Same-process A/B against the per-lane form
// (3 rounds, one box): config 1 +22%, config 2 +8.9%, config-5 buffers +2.5%,
// with amsgrad +4.2% (800 x 265,484 rows: +4.2%); two packs for amsgrad gave
// +2.4% at config 2 and -0.7% on the config-5 buffers. The wavefront form lost
// 1-9% for 16-bit parameters and bfloat16 moments (their load schedules moved),
// so only float32 state takes it.
// Opaque packs (kOpaquePacks / kOpaquePacksPre) in the same A/B: bfloat16
// Adam with a workspace +1.2%, bfloat16 Adagrad with one +0.7-1.0%, float16
// Adagrad without one +5.8%; other combinations of the 16-bit policies moved
// -3% to +1% with them (float32 -3% at configs 1 and 2) and do without.

// Adam / AdamW: h = {lr, beta1, beta2, eps, weight_decay}.
template <typename T_, bool ADAMW, bool AMSGRAD, typename S_ = T_>
struct AdamPolicy {
  using T = T_;
  using S = S_;
  using M = op_t<T>;
  static constexpr int NS = AMSGRAD ? 3 : 2;
  static constexpr uint32_t kStreamLds = residency_lds<T, S>(AMSGRAD ? 12 : 10);
  static constexpr int kStreamUnroll = stream_unroll<T, S>(AMSGRAD ? 1 : 2, 4, 4, 2);
  // float16 Adam (no amsgrad): one 8-element pack under a cap of 20. Three
  // boxes, config-5 shape: 6.16-6.38 TB/s on synthetic moments and
  // 6.37 on moments that start at zero and underflow (the bench's data),
  // against 5.87-6.35 for the uncapped pack, whose rate swung by up to 6%
  // between processes; four packs under a cap of 12 matched it on synthetic
  // moments (6.26-6.40) and lost 1.5% on the zeroed ones.
  static constexpr bool kHalfShape = kHalfAll<T, S> && !AMSGRAD;
  static constexpr bool kBf16ParamShape =
      std::is_same<T, bf16_t>::value && std::is_same<S, bf16_t>::value && !AMSGRAD;
  // float64 Adam with a workspace: one 4-element pack under a cap of 12, the
  // flag read through the scalar cache. Same-process A/B, 64 x 4M doubles, 4
  // rounds: 5.33 TB/s against 5.15 for two packs uncapped with the vector read
  // (one pack uncapped 5.28, under 16 5.26; two packs under 12 5.13; four
  // uncapped 5.09); with amsgrad (64 x 3M) +1.7%. Without a workspace the
  // scalar read: +1%. 16-bit Adam with amsgrad kept its uncapped pack (caps
  // 16 / 20 within 0.8%).
  static constexpr bool kWideShape = std::is_same<T, double>::value;
  static constexpr uint32_t kStreamLdsPre =
      kBf16State<T, S>  ? lds_for_residency(16)
      : kHalfShape      ? lds_for_residency(20)
      : kBf16ParamShape ? lds_for_residency(16)
      : kWideShape      ? lds_for_residency(12)
                        : residency_lds<T, S>(12);
  static constexpr uint32_t kStreamLdsMid =
      kFp32State<T, S> ? lds_for_residency(AMSGRAD ? 12 : 14) : kStreamLdsPre;
  static constexpr int kStreamUnrollPre = stream_unroll<T, S>(1, 1, 1, kWideShape ? 1 : 2);
  static constexpr bool kScalarMask = true;
  static constexpr bool kWavePrologue = kFp32State<T, S>;
  static constexpr bool kOpaquePacksPre = kBf16ParamShape;
  // MALL-resident launches of 16-bit params and bfloat16 moments: one pack,
  // the flag read through the scalar cache (same-process A/B at config 1's
  // shape, 200 calls x 4 rounds: float16 / bfloat16 params +27% / +32%,
  // bfloat16 moments +19% against four packs with the vector read; two packs
  // +10-18%; the scalar read alone +-0.6%). float64 kept its two packs (+-1%).
  static constexpr int kStreamUnrollSmall = stream_unroll<T, S>(2, 1, 1, 2);
  static constexpr bool kScalarMaskSmall =
      !kFp32State<T, S> && !std::is_same<T, double>::value;
  static constexpr int64_t kStreamSmallBytes = kMallBytes;
  static constexpr int kStreamPack = stream_pack<T, S>();
  static constexpr int kSegmentUnroll = stream_unroll<T, S>(2, 4, 4, 2);
  static constexpr int kSegmentThreads = kThreads;
  // With a workspace, every type runs one-wavefront workgroups: one 16-byte
  // pack per thread (two for float64). Measured with 4-element packs (two for
  // 16-bit params, the same bytes per thread as one 8-element pack now), in a
  // same-process A/B on config 5's twelve per-parameter gradients, 4 rounds,
  // against 128 threads x 4 / 8 packs with the vector flag read: bfloat16
  // moments 6.20 TB/s against 5.54, float16 / bfloat16 params 5.93 / 6.18
  // against 5.68 / 5.66 (128 threads x 2 / 4: 5.87 / 6.07 and 5.88 / 5.82);
  // the 8-element pack then +1.4% / +2.4%. float64: two 4-element packs +1.6%
  // against 128 threads x 2, two 2-element packs +15.6% more.
  static constexpr int kSegmentThreadsPre = kStreamThreads;
  static constexpr int kSegmentUnrollPre = std::is_same<T, double>::value ? 2 : 1;
  // float32 Adam's segmented update with a workspace: the flag read through
  // the scalar cache under a cap of 20 (config 5, twelve per-parameter
  // gradients, 3 rounds: 6.35 TB/s against 6.13 for the vector read
  // uncapped; the vector read under cap 20: 6.28). The other types read it
  // scalar too.
  static constexpr bool kSegmentScalarMask = true;
  static constexpr uint32_t kSegmentLdsPre = kFp32State<T, S> ? lds_for_residency(20) : 0u;
  static constexpr bool kLateStores = !AMSGRAD && std::is_same<T_, float>::value;
  static constexpr bool kVariant = false;
  static constexpr int kPreWords = 2;
  struct Rep {
    AdamHyper h;
    AdamConsts<M> c;
  };
  // The step size and sqrt(v)'s divisor of the bumped step (adam_consts).
  __device__ static AdamConsts<M> consts(const Vectors<T>& v, uint32_t r) {
    M bc1, bc2s;
    adam_bias_corrections<M>(hyper_at(v.h[1], r), hyper_at(v.h[2], r), hyper_at(v.steps, r),
                             bc1, bc2s);
    return adam_consts<M>(hyper_at(v.h[0], r), bc1, bc2s);
  }
  __device__ static void precompute(const Vectors<T>& v, uint32_t r, double* out) {
    const AdamConsts<M> c = consts(v, r);
    out[0] = static_cast<double>(c.step_size);
    out[1] = c.bc2s_div;
  }
  template <bool PRE>
  __device__ static void prologue(const Vectors<T>& v, uint32_t r, Rep& rep) {
    hypers(v, r, rep);
    if constexpr (PRE) {
      rep.c.step_size = static_cast<M>(v.pre[kPreStride * r]);
      rep.c.bc2s_div = v.pre[kPreStride * r + 1];
    } else {
      rep.c = consts(v, r);
    }
  }
  // prologue<false> for a replica that every lane of the wavefront shares.
  // The two bias corrections' pow run as one, beta1's on even lanes and
  // beta2's on odd ones, and so do the step size's divide and (float math)
  // the divide that gives sqrt(v)'s divisor; lanes 0 and 1 then hand their
  // values to the whole wavefront. Each value comes from the same operations
  // on the same operands as in consts(), so the bits are the same, at about
  // half of consts()'s fp64 instructions.
  __device__ static void wave_prologue(const Vectors<T>& v, uint32_t r, Rep& rep) {
    hypers(v, r, rep);
    const bool odd = (__lane_id() & 1) != 0;
    const double bc = adam_bias_correction(odd ? rep.h.beta2 : rep.h.beta1,
                                           static_cast<float>(hyper_at(v.steps, r)));
    if constexpr (std::is_same<M, float>::value) {
      // Even lanes: lr / bias_correction1; odd lanes: 1 / bias_correction2_sqrt,
      // each correction narrowed to float first (adam_consts).
      const double den = static_cast<double>(static_cast<float>(odd ? std::sqrt(bc) : bc));
      const double q = (odd ? 1.0 : rep.h.lr) / den;
      rep.c.step_size = static_cast<float>(wave_lane(q, 0));
      rep.c.bc2s_div = wave_lane(q, 1);
    } else {
      const double x = odd ? std::sqrt(bc) : rep.h.lr / bc;
      rep.c.step_size = wave_lane(x, 0);
      rep.c.bc2s_div = wave_lane(x, 1);
    }
  }
  __device__ static void hypers(const Vectors<T>& v, uint32_t r, Rep& rep) {
    rep.h.lr = hyper_at(v.h[0], r);
    rep.h.beta1 = hyper_at(v.h[1], r);
    rep.h.beta2 = hyper_at(v.h[2], r);
    rep.h.eps = hyper_at(v.h[3], r);
    rep.h.weight_decay = hyper_at(v.h[4], r);
  }
  __device__ static bool reads_state(const Vectors<T>&, uint32_t) { return true; }
  __device__ static bool decays(const Rep& rep) { return rep.h.weight_decay != 0; }
  __device__ static void drop_decay(Rep& rep) { rep.h.weight_decay = 0.0; }
  __device__ static void update(M& p, M g, M (&s)[NS], const Rep& rep, bool maximize) {
    M mx = M(0);
    if constexpr (AMSGRAD) mx = s[2];
    adam_element<M, ADAMW, AMSGRAD, std::is_same<S, _Float16>::value>(p, g, s[0], s[1], mx,
                                                                      rep.h, maximize, rep.c);
    if constexpr (AMSGRAD) s[2] = mx;
  }
};

// SGD: h = {lr, momentum, dampening, weight_decay}. The hyperparameters are
// carried as double inside the element math, as torch's ROCm `_fused_sgd_`
// takes them (checked on the MI355X: carrying them as float instead changes
// params and buffers by up to a few ulp). Its prologue is four loads and a
// compare: nothing to precompute.
template <typename T_, bool HAS_BUF, bool NESTEROV, typename S_ = T_>
struct SgdPolicy {
  using T = T_;
  using S = S_;
  using M = op_t<T>;
  static constexpr int NS = HAS_BUF ? 1 : 0;
  // bfloat16 params and momentum buffers: two 8-element packs under a cap of
  // 20. Two boxes, two processes each, config-5 shape: 6.19-6.45 TB/s against
  // 6.07-6.34 for one uncapped pack.
  static constexpr bool kBf16Shape =
      HAS_BUF && std::is_same<T, bf16_t>::value && std::is_same<S, bf16_t>::value;
  static constexpr uint32_t kStreamLds =
      kBf16Shape ? lds_for_residency(20) : HAS_BUF ? residency_lds<T, S>(20) : 0u;
  // float64 with momentum: one 4-element pack, uncapped, the flag read
  // through the scalar cache (same-process A/B on 64 x 4M doubles: +3.4%
  // against two packs with the vector read; under a cap of 12: -5%).
  // float32 without momentum: one pack, uncapped, the scalar read (same-process
  // A/B, 4 rounds, config-5 buffers: 6.46 TB/s against 5.38 for two packs with
  // the vector read; two packs with the scalar read 5.59, four 6.07, one pack
  // under a cap of 20 6.06; its MALL-resident launches +2.3% with the scalar
  // read at config 3's size).
  static constexpr int kStreamUnroll =
      kBf16Shape ? 2 : stream_unroll<T, S>(1, 1, 1, HAS_BUF ? 1 : 2);
  static constexpr uint32_t kStreamLdsPre = kStreamLds;
  static constexpr uint32_t kStreamLdsMid = kStreamLdsPre;
  static constexpr int kStreamUnrollPre = kStreamUnroll;
  static constexpr int kStreamUnrollSmall = stream_unroll<T, S>(1, 1, 4, 2);
  static constexpr bool kScalarMask =
      std::is_same<T, float>::value || (HAS_BUF && std::is_same<T, double>::value);
  static constexpr bool kScalarMaskSmall = kScalarMask;
  // float32 launches that fit the MALL: four-wavefront workgroups. Config 3's
  // shape (32 x 545100, 80% active) with the vector flag read, two calls, 2-3
  // processes: 128 threads 6.87-6.91 TB/s against 6.77-6.79 for one wavefront
  // and 6.88-6.93 for 256; with the scalar read 256 threads ran 2.2% ahead of
  // 128 (same-process A/B, 10 rounds).
  static constexpr int kStreamBlockSmall = kFp32State<T, S> ? 256 : kStreamThreads;
  static constexpr int64_t kStreamSmallBytes = kMallBytes;
  static constexpr int kStreamPack = stream_pack<T, S>();
  // Segmented float32 updates: one-wavefront workgroups, one pack, the flag
  // read through the scalar cache (same-process A/B on config 5's twelve
  // per-parameter gradients, 4 rounds: 6.28 TB/s against 5.95 for 128 threads
  // x 2 packs with the vector read; 128 x 1: 6.19). 16-bit: one wavefront x 8
  // elements, scalar read (as two 4-element packs: float16 / bfloat16 6.33 /
  // 6.29 against 5.76 / 5.71; 4 elements 5.46 / 5.37, 16 5.92 / 5.91).
  // bfloat16 state: one pack, +2.5% (two: -10%); float64: two 2-element packs
  // (+15.5% against two 4-element ones).
  static constexpr int kSegmentUnroll = std::is_same<T, double>::value ? 2 : 1;
  static constexpr int kSegmentThreads = kStreamThreads;
  static constexpr int kSegmentThreadsPre = kThreads;
  static constexpr int kSegmentUnrollPre = kSegmentUnroll;
  static constexpr bool kSegmentScalarMask = true;
  static constexpr bool kLateStores = std::is_same<T_, float>::value;
  static constexpr bool kVariant = false;
  static constexpr int kPreWords = 0;
  struct Rep {
    SgdHyper<double> h;
    bool first;
  };
  __device__ static void precompute(const Vectors<T>&, uint32_t, double*) {}
  template <bool PRE>
  __device__ static void prologue(const Vectors<T>& v, uint32_t r, Rep& rep) {
    rep.h.lr = hyper_at(v.h[0], r);
    rep.h.momentum = hyper_at(v.h[1], r);
    rep.h.dampening = hyper_at(v.h[2], r);
    rep.h.weight_decay = hyper_at(v.h[3], r);
    rep.first = widen(v.steps[r]) == M(1);
  }
  // On a replica's first step the buffer is overwritten by the gradient
  // without being read, so it is not fetched.
  __device__ static bool reads_state(const Vectors<T>& v, uint32_t r) {
    return widen(v.steps[r]) != M(1);
  }
  __device__ static bool decays(const Rep& rep) { return rep.h.weight_decay != 0; }
  __device__ static void drop_decay(Rep& rep) { rep.h.weight_decay = 0.0; }
  __device__ static void update(M& p, M g, M (&s)[NS > 0 ? NS : 1], const Rep& rep,
                                bool maximize) {
    M buf = s[0];
    sgd_element<M, double, HAS_BUF, NESTEROV>(p, g, buf, rep.h, maximize, rep.first);
    s[0] = buf;
  }
};

// Adagrad: h = {lr, lr_decay, weight_decay, eps}.
template <typename T_, typename S_ = T_>
struct AdagradPolicy {
  using T = T_;
  using S = S_;
  using M = op_t<T>;
  static constexpr int NS = 1;
  static constexpr uint32_t kStreamLds = residency_lds<T, S>(16);
  // float64: one 4-element pack, uncapped, the scalar flag read (same-process
  // A/B on 64 x 4M doubles against two packs with the vector read: +2.1% with
  // a workspace, +1.3% without; under a cap of 12: -3% / -5%).
  static constexpr int kStreamUnroll = stream_unroll<T, S>(1, 1, 1, 1);
  static constexpr uint32_t kStreamLdsPre =
      kBf16State<T, S> ? lds_for_residency(20) : residency_lds<T, S>(14);
  static constexpr uint32_t kStreamLdsMid = kStreamLdsPre;
  static constexpr int kStreamUnrollPre = stream_unroll<T, S>(1, 1, 4, 1);
  static constexpr bool kScalarMask =
      std::is_same<T, float>::value || std::is_same<T, double>::value;
  static constexpr bool kOpaquePacks = kHalfAll<T, S>;
  static constexpr bool kOpaquePacksPre =
      std::is_same<T, bf16_t>::value && std::is_same<S, bf16_t>::value;
  // MALL-resident 16-bit launches: one pack, the scalar flag read (at config
  // 4's shape against four packs with the vector read: bfloat16 +12%, float16
  // +9%; two packs +5%).
  static constexpr int kStreamUnrollSmall = stream_unroll<T, S>(2, 1, 1, 2);
  static constexpr bool kScalarMaskSmall = sizeof(T) == 2;
  static constexpr int64_t kStreamSmallBytes = kMallBytes;
  static constexpr int kStreamPack = stream_pack<T, S>();
  // Segmented float32 updates with a workspace: one-wavefront workgroups, one
  // pack, the scalar flag read, uncapped (same-process A/B on config 5's
  // twelve per-parameter gradients, 4 rounds: 6.34 TB/s against 5.97 for 128
  // threads x 2 packs with the vector read; under a cap of 20: 6.13). Without
  // a workspace the shape stays; the scalar read costs it 0.5%. 16-bit with a
  // workspace: one wavefront x 16 elements, scalar read (as four 4-element
  // packs: float16 / bfloat16 5.76 / 5.73 against 5.39 / 5.46; 8 elements 5.49
  // / 5.62, 4 4.70 / 4.95; as two 8-element packs +2.3% / +4% more).
  // bfloat16 state: one pack, +2.4% (two: -10%); float64: two 2-element packs.
  static constexpr int kSegmentUnroll = sizeof(T) == 2 ? 1 : 2;
  static constexpr int kSegmentThreads = kThreads;
  static constexpr int kSegmentThreadsPre = kStreamThreads;
  static constexpr int kSegmentUnrollPre =
      kFp32State<T, S> || kBf16State<T, S> ? 1 : 2;
  static constexpr bool kSegmentScalarMask = true;
  static constexpr bool kLateStores = false;
  static constexpr bool kVariant = std::is_same_v<T, _Float16> && std::is_same_v<S, _Float16>;
  static constexpr int kPreWords = 1;
  struct Rep {
    AdagradHyper h;
    bool once;  // float16 state sum rounded once (ilp_row)
  };
  // corrected_lr of the bumped step.
  __device__ static void precompute(const Vectors<T>& v, uint32_t r, double* out) {
    out[0] = adagrad_corrected_lr(hyper_at(v.h[0], r), hyper_at(v.h[1], r),
                                  static_cast<float>(widen(v.steps[r])));
  }
  template <bool PRE>
  __device__ static void prologue(const Vectors<T>& v, uint32_t r, Rep& rep) {
    rep.h.weight_decay = hyper_at(v.h[2], r);
    rep.h.eps = hyper_at(v.h[3], r);
    rep.once = kVariant && ilp_row(v.ilp_rows, r);
    if constexpr (PRE) {
      rep.h.corrected_lr = v.pre[kPreStride * r];
    } else {
      rep.h.corrected_lr = adagrad_corrected_lr(hyper_at(v.h[0], r), hyper_at(v.h[1], r),
                                                static_cast<float>(widen(v.steps[r])));
    }
  }
  __device__ static bool reads_state(const Vectors<T>&, uint32_t) { return true; }
  __device__ static bool decays(const Rep& rep) { return rep.h.weight_decay != 0; }
  __device__ static void drop_decay(Rep& rep) { rep.h.weight_decay = 0.0; }
  // float16 parameters and state. torch's fused Adagrad stores the state sum
  // of a row on its vector path (ilp_row) rounded once from the exact
  // g * g + s, g the maximized and decayed gradient (its build turns the float
  // fma and the narrowing into one v_fma_mix); on its element path it stores
  // the float sum, which the square root takes everywhere, rounded to half.
  // The two differ where g * g + s lies within a quarter of a float ulp of a
  // half-way point between two halves without being one (such as a half-way
  // g * g and a float16 subnormal s). The once-rounded form agrees with torch
  // on every pair of float16 (g, s) values, maximize either way; bfloat16 and
  // the other types store the rounded float sum on both paths.
  __device__ static bool variant(const Rep& rep) { return rep.once; }
  __device__ static void set_variant(Rep& rep, bool once) { rep.once = once; }
  // A pack on a vector-path row (false otherwise, for the generic form): the
  // update as apply_pack's, then the state pairs straight out of
  // v_fma_mixlo/hi_f16 on the decayed gradients and the sums as loaded, in
  // place of narrowing the float sums (one instruction more per pair).
  template <int N>
  __device__ static bool update_pack(Pack<T, N>& vp, const Pack<T, N>& vg, Pack<S, N>& vs,
                                     const Rep& rep, bool maximize) {
    static_assert(N % 2 == 0, "state pairs");
    if (!rep.once) return false;
    struct Words {
      uint32_t w[N / 2];
    };
    const Words s_in = __builtin_bit_cast(Words, vs);
    M pm[N], gm[N], sm[N];
#pragma unroll
    for (int e = 0; e < N; ++e) {
      pm[e] = widen(vp.v[e]);
      gm[e] = widen(vg.v[e]);
      sm[e] = widen(vs.v[e]);
    }
#pragma unroll
    for (int e = 0; e < N; ++e) {
      adagrad_sum<M>(pm[e], gm[e], sm[e], rep.h, maximize);
      adagrad_finish<M>(pm[e], gm[e], sqrt_rn<true>(sm[e]), rep.h);
    }
    Words out;
#pragma unroll
    for (int k = 0; k < N / 2; ++k) {
      out.w[k] = fma_half2_sq(gm[2 * k], gm[2 * k + 1], s_in.w[k]);
    }
    vs = __builtin_bit_cast(Pack<S, N>, out);
#pragma unroll
    for (int e = 0; e < N; ++e) vp.v[e] = narrow<T>(pm[e]);
    return true;
  }
  __device__ static void update(M& p, M g, M (&s)[NS], const Rep& rep, bool maximize) {
    if constexpr (kVariant) {
      if (rep.once) {
        const M s_in = s[0];
        adagrad_sum<M>(p, g, s[0], rep.h, maximize);
        adagrad_finish<M>(p, g, sqrt_rn<true>(s[0]), rep.h);
        s[0] = fma_half(g, g, s_in);
        return;
      }
    }
    adagrad_element<M, std::is_same<S, _Float16>::value>(p, g, s[0], rep.h, maximize);
  }
};

// Float32 Adagrad (TS_ADAGRAD_F32): the reference CPU kernel's float element
// math instead of ATen's fp64 update; h = {lr, lr_decay, wd, eps}. The math
// type is float for every storage type (float64 parameters are rejected).
template <typename T_, typename S_ = T_>
struct AdagradF32Policy {
  using T = T_;
  using S = S_;
  using M = float;
  static constexpr int NS = 1;
  // With the scalar flag read, as the fp64-math Adagrad: one pack under cap
  // 14 with a workspace, one pack under 16 without (same-process A/B against
  // the vector read at cap 20 / two packs, 6 rounds: config 4 +1.8%, config-5
  // buffers +1.8%, without a workspace +5.7-7.0%).
  static constexpr uint32_t kStreamLds = residency_lds<T, S>(16);
  static constexpr int kStreamUnroll = stream_unroll<T, S>(1, 1, 1, 2);
  static constexpr uint32_t kStreamLdsPre = residency_lds<T, S>(14);
  static constexpr uint32_t kStreamLdsMid = kStreamLdsPre;
  static constexpr int kStreamUnrollPre = stream_unroll<T, S>(1, 1, 1, 2);
  static constexpr bool kScalarMask = std::is_same<T, float>::value;
  static constexpr int kStreamUnrollSmall = stream_unroll<T, S>(2, 1, 4, 2);
  static constexpr int64_t kStreamSmallBytes = kMallBytes;
  static constexpr int kStreamPack = stream_pack<T, S>();
  // Segmented with a workspace: one-wavefront workgroups, one pack, the
  // scalar flag read, as Adagrad (config 5's per-parameter gradients,
  // same-process A/B: +6.1%; without a workspace the scalar read -0.6%).
  static constexpr int kSegmentUnroll = 2;
  static constexpr int kSegmentThreads = kThreads;
  static constexpr int kSegmentThreadsPre = kStreamThreads;
  static constexpr int kSegmentUnrollPre = 1;
  static constexpr bool kSegmentScalarMask = true;
  static constexpr bool kLateStores = false;
  static constexpr bool kVariant = false;
  static constexpr int kPreWords = 1;
  struct Rep {
    AdagradF32Hyper h;
  };
  __device__ static void precompute(const Vectors<T>& v, uint32_t r, double* out) {
    out[0] = static_cast<double>(
        adagrad_corrected_lr_f32(hyper_at(v.h[0], r), hyper_at(v.h[1], r), hyper_at(v.steps, r)));
  }
  template <bool PRE>
  __device__ static void prologue(const Vectors<T>& v, uint32_t r, Rep& rep) {
    const double wd = hyper_at(v.h[2], r);
    rep.h.weight_decay = static_cast<float>(wd);
    rep.h.has_weight_decay = wd != 0.0;
    rep.h.eps = static_cast<float>(hyper_at(v.h[3], r));
    if constexpr (PRE) {
      rep.h.corrected_lr = static_cast<float>(v.pre[kPreStride * r]);
    } else {
      rep.h.corrected_lr = adagrad_corrected_lr_f32(hyper_at(v.h[0], r), hyper_at(v.h[1], r),
                                                    hyper_at(v.steps, r));
    }
  }
  __device__ static bool reads_state(const Vectors<T>&, uint32_t) { return true; }
  __device__ static bool decays(const Rep& rep) { return rep.h.has_weight_decay; }
  __device__ static void drop_decay(Rep& rep) {
    rep.h.weight_decay = 0.0f;
    rep.h.has_weight_decay = false;
  }
  __device__ static void update(M& p, M g, M (&s)[NS], const Rep& rep, bool maximize) {
    adagrad_element_f32(p, g, s[0], rep.h, maximize);
  }
};

template <typename P>
constexpr int state_slots() {
  return P::NS > 0 ? P::NS : 1;
}

// Packs per thread and residency reservation of the streaming driver, with
// the per-replica constants read from a workspace (PRE) or derived in every
// workgroup, for large launches and for SMALL ones (operands that fit the
// MALL: plain accesses, no cap).
template <typename P, bool PRE, bool SMALL>
constexpr int stream_unroll_of() {
  return SMALL ? P::kStreamUnrollSmall : PRE ? P::kStreamUnrollPre : P::kStreamUnroll;
}
template <typename P, bool PRE, bool SMALL>
constexpr uint32_t stream_lds_of() {
  return SMALL ? 0u : PRE ? P::kStreamLdsPre : P::kStreamLds;
}

// Threads per streaming workgroup: one wavefront, or a policy's kStreamBlock
// for its launches beyond the MALL and kStreamBlockSmall for the others.
template <typename P, typename = void>
struct stream_block_of {
  static constexpr int value = kStreamThreads;
};
template <typename P>
struct stream_block_of<P, std::void_t<decltype(P::kStreamBlock)>> {
  static constexpr int value = P::kStreamBlock;
};
template <typename P, typename = void>
struct stream_block_small_of {
  static constexpr int value = kStreamThreads;
};
template <typename P>
struct stream_block_small_of<P, std::void_t<decltype(P::kStreamBlockSmall)>> {
  static constexpr int value = P::kStreamBlockSmall;
};
template <typename P, bool SMALL>
constexpr int stream_threads() {
  return SMALL ? stream_block_small_of<P>::value : stream_block_of<P>::value;
}

// How a streaming workgroup reads its replica's active flag: through the
// scalar cache (mask_byte_scalar) or with a vector load. The scalar read skips
// the vector memory pipeline, which the streaming loads keep queued, so a
// workgroup starts its loads sooner and a frozen replica's workgroup exits
// sooner; the residency caps below are tuned with it. By default launches
// beyond the MALL read it scalar and SMALL ones as a vector load
// (kScalarMask / kScalarMaskSmall override).
template <typename P, typename = void>
struct scalar_mask_of {
  static constexpr bool value = true;
};
template <typename P>
struct scalar_mask_of<P, std::void_t<decltype(P::kScalarMask)>> {
  static constexpr bool value = P::kScalarMask;
};
template <typename P, typename = void>
struct scalar_mask_small_of {
  static constexpr bool value = false;
};
template <typename P>
struct scalar_mask_small_of<P, std::void_t<decltype(P::kScalarMaskSmall)>> {
  static constexpr bool value = P::kScalarMaskSmall;
};
template <typename P, bool SMALL>
constexpr bool stream_scalar_mask() {
  return SMALL ? scalar_mask_small_of<P>::value : scalar_mask_of<P>::value;
}

// A policy's constants for a replica that a whole workgroup works on: its
// `wave_prologue` (derived once per wavefront, the work spread over lanes)
// where it sets kWavePrologue and the constants are derived, else
// `prologue<PRE>`. Every lane of the wavefront must be active.
template <typename P, typename = void>
struct wave_prologue_of {
  static constexpr bool value = false;
};
template <typename P>
struct wave_prologue_of<P, std::void_t<decltype(P::kWavePrologue)>> {
  static constexpr bool value = P::kWavePrologue;
};
template <typename P, bool PRE>
__device__ __forceinline__ void uniform_prologue(const Vectors<typename P::T>& v, uint32_t r,
                                                 typename P::Rep& rep) {
  if constexpr (!PRE && wave_prologue_of<P>::value) {
    P::wave_prologue(v, r, rep);
  } else {
    P::template prologue<PRE>(v, r, rep);
  }
}

// Whether the streaming driver's large launches start a thread's packs from
// opaque values (opaque()) rather than undefined ones: P::kOpaquePacks without
// a workspace, P::kOpaquePacksPre with one; by default not. It changes the
// compiler's schedule of the loads, and that pays for some 16-bit policies and
// costs others (the policies say which).
template <typename P, typename = void>
struct opaque_packs_of {
  static constexpr bool value = false;
};
template <typename P>
struct opaque_packs_of<P, std::void_t<decltype(P::kOpaquePacks)>> {
  static constexpr bool value = P::kOpaquePacks;
};
template <typename P, typename = void>
struct opaque_packs_pre_of {
  static constexpr bool value = false;
};
template <typename P>
struct opaque_packs_pre_of<P, std::void_t<decltype(P::kOpaquePacksPre)>> {
  static constexpr bool value = P::kOpaquePacksPre;
};
template <typename P, bool PRE, bool SMALL>
constexpr bool stream_opaque_packs() {
  return !SMALL && (PRE ? opaque_packs_pre_of<P>::value : opaque_packs_of<P>::value);
}

// The segmented driver's flag read and residency reservation with a
// workspace (kSegmentScalarMask / kSegmentLdsPre; by default a vector load,
// uncapped).
template <typename P, typename = void>
struct segment_scalar_mask_of {
  static constexpr bool value = false;
};
template <typename P>
struct segment_scalar_mask_of<P, std::void_t<decltype(P::kSegmentScalarMask)>> {
  static constexpr bool value = P::kSegmentScalarMask;
};
template <typename P, typename = void>
struct segment_lds_pre_of {
  static constexpr uint32_t value = 0;
};
template <typename P>
struct segment_lds_pre_of<P, std::void_t<decltype(P::kSegmentLdsPre)>> {
  static constexpr uint32_t value = P::kSegmentLdsPre;
};

// Replica r's active flag through the scalar cache: one s_load_dword of the
// aligned dword that holds byte r (that dword never leaves the page the byte
// is on), then the byte. The address is uniform over the workgroup. The
// scalar and vector L1 caches are invalidated between kernel dispatches, so a
// mask written before the launch is what the load sees.
__device__ __forceinline__ bool mask_byte_scalar(const uint8_t* mask, uint32_t r) {
  const uintptr_t at = reinterpret_cast<uintptr_t>(mask) + r;
  const auto* word =
      reinterpret_cast<const __attribute__((address_space(4))) uint32_t*>(at & ~uintptr_t(3));
  return ((*word >> (8 * (at & 3))) & 0xFFu) != 0;
}

// Elements per streaming tile: the workgroup's threads x the policy's packs
// per thread.
template <typename P, bool PRE, bool SMALL>
constexpr int64_t stream_tile() {
  return int64_t(stream_threads<P, SMALL>()) * P::kStreamPack * stream_unroll_of<P, PRE, SMALL>();
}

// Bytes of (R, T) operands a launch reads (all rows): params and grads in
// the parameter type, the state buffers in the state type.
template <typename P>
constexpr int64_t operand_bytes_per_elem() {
  return 2 * int64_t(sizeof(typename P::T)) + P::NS * int64_t(sizeof(typename P::S));
}

// Workgroup size, packs per thread and elements per tile of the segmented
// driver, with the per-replica constants read from a workspace (PRE) or
// derived in every workgroup. Measured per policy at the config-5 layout with
// per-parameter gradients (128 threads, 1/2/4 packs): Adam with bfloat16
// moments or 16-bit params wants 4 (+8-17%); SGD and Adagrad were within noise
// of 2 for every operand type, and float32/float64 Adam too. With
// one-instruction bfloat16 narrowing, 16-bit Adam gained again from 8: +2.7%
// (half), +4.2% (bfloat16). Float32 Adam with a workspace takes the dense
// update's one-wave workgroups with one pack, uncapped: on one box 6.33 TB/s
// against 6.03 for the previous 128 threads x 2 packs under a cap of 8
// workgroups per CU (64 or 128 threads x 1 or 2 packs x caps 6-20 and none, 3
// interleaved rounds); on another, 5 rounds, every one of those shapes within
// 0.2% (6.33-6.35, also when the gradient is stored on the way), 1.6% behind
// the dense update on the same buffers.
template <typename P, bool PRE>
constexpr int segment_threads() {
  return PRE ? P::kSegmentThreadsPre : P::kSegmentThreads;
}
template <typename P, bool PRE>
constexpr int segment_unroll() {
  return PRE ? P::kSegmentUnrollPre : P::kSegmentUnroll;
}
template <typename P, bool PRE>
constexpr int64_t segment_tile() {
  return int64_t(segment_threads<P, PRE>()) * stream_pack<typename P::T, typename P::S>() *
         segment_unroll<P, PRE>();
}

template <typename P>
struct KArgs {
  Operands<typename P::T> x;
  Vectors<typename P::T> vec;
  Grid g;
  bool maximize;
};

// One element through the policy: widen, update, narrow. `s_io` holds the
// state operands' values (unread ones are never used).
template <typename P>
__device__ __forceinline__ void apply_element(typename P::T& p_io, typename P::T g_in,
                                              typename P::S (&s_io)[state_slots<P>()],
                                              bool load_state, const typename P::Rep& rep,
                                              bool maximize) {
  using M = typename P::M;
  M p = widen(p_io);
  M s[state_slots<P>()];
#pragma unroll
  for (int k = 0; k < state_slots<P>(); ++k) {
    s[k] = (load_state && k < P::NS) ? M(widen(s_io[k])) : M(0);
  }
  P::update(p, widen(g_in), s, rep, maximize);
  p_io = narrow<typename P::T>(p);
#pragma unroll
  for (int k = 0; k < P::NS; ++k) {
    s_io[k] = narrow<typename P::S>(s[k]);
  }
}

// N math-type values narrowed into a pack: bfloat16 two at a time
// (narrow2_bf16, the same bits as narrow<bf16_t> per value), every other type
// one at a time (hipcc pairs the half conversions itself).
template <typename T, int N>
__device__ __forceinline__ Pack<T, N> narrow_pack(const op_t<T> (&x)[N]) {
  if constexpr (std::is_same<T, bf16_t>::value && N % 2 == 0) {
    struct Words {
      uint32_t w[N / 2];
    } out;
#pragma unroll
    for (int k = 0; k < N / 2; ++k) out.w[k] = narrow2_bf16(x[2 * k], x[2 * k + 1]);
    return __builtin_bit_cast(Pack<T, N>, out);
  } else {
    Pack<T, N> out;
#pragma unroll
    for (int k = 0; k < N; ++k) out.v[k] = narrow<T>(x[k]);
    return out;
  }
}

// A pack of N elements through the policy, as apply_element does one: widen,
// update, narrow (the whole pack at once). `vs` holds the state operands'
// packs (unread ones are never used).
template <typename P, int N>
__device__ __forceinline__ void apply_pack(Pack<typename P::T, N>& vp,
                                           const Pack<typename P::T, N>& vg,
                                           Pack<typename P::S, N> (&vs)[state_slots<P>()],
                                           bool load_state, const typename P::Rep& rep,
                                           bool maximize) {
  using M = typename P::M;
  constexpr int SS = state_slots<P>();
  if constexpr (P::kVariant) {
    if (P::template update_pack<N>(vp, vg, vs[0], rep, maximize)) return;
  }
  M pm[N], gm[N];
  M sm[SS][N];
#pragma unroll
  for (int e = 0; e < N; ++e) {
    pm[e] = widen(vp.v[e]);
    gm[e] = widen(vg.v[e]);
#pragma unroll
    for (int k = 0; k < SS; ++k) {
      sm[k][e] = (load_state && k < P::NS) ? M(widen(vs[k].v[e])) : M(0);
    }
  }
#pragma unroll
  for (int e = 0; e < N; ++e) {
    M s[SS];
#pragma unroll
    for (int k = 0; k < SS; ++k) s[k] = sm[k][e];
    P::update(pm[e], gm[e], s, rep, maximize);
#pragma unroll
    for (int k = 0; k < SS; ++k) sm[k][e] = s[k];
  }
  vp = narrow_pack<typename P::T, N>(pm);
#pragma unroll
  for (int k = 0; k < P::NS; ++k) vs[k] = narrow_pack<typename P::S, N>(sm[k]);
}

// Row r of (R, T) operand b, as the parameter type (b < 2) or the state type.
template <typename P>
__device__ __forceinline__ typename P::T* pg_row(const Operands<typename P::T>& x, int b,
                                                 uint32_t r) {
  return x.data[b] + int64_t(r) * x.stride_r[b];
}
template <typename P>
__device__ __forceinline__ typename P::S* state_row(const Operands<typename P::T>& x, int b,
                                                    uint32_t r) {
  return reinterpret_cast<typename P::S*>(x.data[b]) + int64_t(r) * x.stride_r[b];
}

// Runs `f` on the replica's constants with the policy's variant choice, if it
// has one, set to a literal: one branch per workgroup, and element math
// compiled for each choice.
template <typename P, typename F>
__device__ __forceinline__ void with_variant(const typename P::Rep& rep, F&& f) {
  if constexpr (P::kVariant) {
    typename P::Rep fixed = rep;
    if (P::variant(rep)) {
      P::set_variant(fixed, true);
      f(fixed);
    } else {
      P::set_variant(fixed, false);
      f(fixed);
    }
  } else {
    f(rep);
  }
}

// Runs `f` with `maximize` as a literal for policies with a variant, whose
// pack form takes the sign-corrected gradient as a value (a run-time flag
// would cost a negation and a select per element there); others get the
// run-time flag.
template <typename P, typename F>
__device__ __forceinline__ void with_maximize(bool maximize, F&& f) {
  if constexpr (P::kVariant) {
    if (maximize) {
      f(true);
    } else {
      f(false);
    }
  } else {
    f(maximize);
  }
}

// ---------------------------------------------------------------------------
// Drivers
// ---------------------------------------------------------------------------
// PRE: the per-replica constants come from the call's workspace (a.vec.pre).
// A thread's loads are issued before the replica's prologue, which then runs
// while they are in flight.
// SMALL: the launch's operands fit the MALL; plain accesses and the small-launch
// tile instead of non-temporal ones.
template <typename P, bool ANY, bool PRE, bool SMALL>
__global__ __launch_bounds__((stream_threads<P, SMALL>())) void stream_kernel(KArgs<P> a) {
  constexpr int NTH = stream_threads<P, SMALL>();  // threads per workgroup
  using T = typename P::T;
  using S = typename P::S;
  constexpr int NS = P::NS;
  constexpr int SS = state_slots<P>();
  constexpr bool NT = !SMALL;
  constexpr int KP = P::kStreamPack;
  constexpr int U = stream_unroll_of<P, PRE, SMALL>();
  constexpr int64_t kStreamTile = stream_tile<P, PRE, SMALL>();
  static_assert((kStreamTile & (kStreamTile - 1)) == 0 &&
                    phase_elems<T>() % kStreamTile == 0,
                "streaming tiles align to their own size, a divisor of the phase modulus");
  uint32_t r;
  int64_t t0;
  stream_tile_of_block<kStreamTile>(a.g, r, t0);
  if constexpr (stream_scalar_mask<P, SMALL>()) {
    if (!mask_byte_scalar(a.vec.mask, r)) return;
  } else {
    if (!a.vec.mask[r]) return;
  }

  // A row's tiles k >= 1 start at its first kStreamTile-element boundary, so
  // no tile straddles one (on rows whose length is not a multiple of the tile,
  // 0.2-1.7% faster than tiles on 256-byte boundaries, measured on the MI355X).
  // Tile 0 takes what lies before that boundary: packs from the first pack
  // boundary, the fewer than KP elements before it one at a time, and the
  // row's fewer than KP tail elements. The two kinds branch apart here, so a
  // main tile computes no more addresses than a plain row-major tile.
  const int64_t width = a.g.T;
  const uint32_t phase = (a.g.res0 + r * a.g.rmod) % uint32_t(kStreamTile);
  const int64_t head = imin(width, (kStreamTile - phase) % kStreamTile);

  // The packs [first, first + packs_left * KP) of row r, then (head tile)
  // the single elements [0, pre) and [body_end, width).
  const auto run = [&](auto head_tile, int64_t first, int64_t packs_left, int64_t pre,
                       int64_t body_end) __attribute__((always_inline)) {
    const bool load_state = P::reads_state(a.vec, r);
    T* const pbase = pg_row<P>(a.x, 0, r);
    const T* const gbase = pg_row<P>(a.x, 1, r);
    S* sbase[SS];
#pragma unroll
    for (int b = 0; b < NS; ++b) sbase[b] = state_row<P>(a.x, 2 + b, r);

    // The parameters' packs are aligned by construction (`first` lies on a
    // pack boundary of the row); with ANY the other operands sit at another
    // phase and use element-aligned packs.
    Pack<T, KP>* prow = reinterpret_cast<Pack<T, KP>*>(pbase + first);
    const Packs<ANY, T, NT, KP> grow(const_cast<T*>(gbase) + first);
    Packs<ANY, S, NT, KP> srow[SS];
#pragma unroll
    for (int b = 0; b < NS; ++b) srow[b] = Packs<ANY, S, NT, KP>(sbase[b] + first);

    Pack<T, KP> vp[U], vg[U];
    Pack<S, KP> vs[SS][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = int64_t(u) * NTH + threadIdx.x;
      if constexpr (stream_opaque_packs<P, PRE, SMALL>()) {
        opaque(vp[u]);
        opaque(vg[u]);
#pragma unroll
        for (int b = 0; b < SS; ++b) opaque(vs[b][u]);
      }
      if (i < packs_left) {
        vp[u] = load_stream<NT>(prow + i);
        vg[u] = grow.load(i);
        if (load_state) {
#pragma unroll
          for (int b = 0; b < NS; ++b) {
            vs[b][u] = srow[b].load(i);
          }
        }
      }
    }
    typename P::Rep rep;
    uniform_prologue<P, PRE>(a.vec, r, rep);
    const auto store_packs = [&](int u, int64_t i) {
      store_stream<NT>(prow + i, vp[u]);
#pragma unroll
      for (int b = 0; b < NS; ++b) {
        srow[b].store(i, vs[b][u]);
      }
    };
    const auto compute = [&](const typename P::Rep& rp, bool maximize)
                             __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = int64_t(u) * NTH + threadIdx.x;
        if (i < packs_left) {
          Pack<S, KP> st[SS];
#pragma unroll
          for (int b = 0; b < NS; ++b) st[b] = vs[b][u];
          apply_pack<P, KP>(vp[u], vg[u], st, load_state, rp, maximize);
#pragma unroll
          for (int b = 0; b < NS; ++b) vs[b][u] = st[b];
          if constexpr (!P::kLateStores) store_packs(u, i);
        }
      }
    };
    // The replica's weight decay and `maximize` are uniform over the workgroup:
    // branch on them once instead of evaluating the decay term per element and
    // selecting (what the compiler makes of the per-element test). The common
    // case, neither, runs the math with both as constants.
    if (!a.maximize && !P::decays(rep)) {
      typename P::Rep plain = rep;
      P::drop_decay(plain);
      with_variant<P>(plain, [&](const typename P::Rep& rp) { compute(rp, false); });
    } else {
      with_variant<P>(rep, [&](const typename P::Rep& rp) {
        with_maximize<P>(a.maximize, [&](bool mx) { compute(rp, mx); });
      });
    }
    if constexpr (P::kLateStores) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = int64_t(u) * NTH + threadIdx.x;
        if (i < packs_left) store_packs(u, i);
      }
    }

    if constexpr (decltype(head_tile)::value) {
      // The elements before the row's first pack boundary and its fewer than
      // KP tail elements, one element per access.
      const auto one = [&](int64_t j) {
        T pe = pbase[j];
        S st[SS];
        if (load_state) {
#pragma unroll
          for (int b = 0; b < NS; ++b) st[b] = sbase[b][j];
        }
        apply_element<P>(pe, gbase[j], st, load_state, rep, a.maximize);
        pbase[j] = pe;
#pragma unroll
        for (int b = 0; b < NS; ++b) sbase[b][j] = st[b];
      };
      for (int64_t j = threadIdx.x; j < pre; j += NTH) one(j);
      for (int64_t j = body_end + threadIdx.x; j < width; j += NTH) one(j);
    }
  };

  if (t0 != 0) {
    const int64_t packs_left = (width - head) / KP - (t0 - kStreamTile) / KP;
    if (packs_left > 0) {
      run(std::false_type{}, head + (t0 - kStreamTile), packs_left, 0, width);
    }
    return;
  }
  const int64_t pre = imin(head, (KP - phase % KP) % KP);
  const int64_t head_packs = (head - pre) / KP;
  const int64_t body_end =
      head < width ? head + (width - head) / KP * KP : pre + head_packs * KP;
  if (head_packs > 0 || pre > 0 || body_end < width) {
    run(std::true_type{}, pre, head_packs, pre, body_end);
  }
}

// The element driver's shape: kElemThreads threads x kElemPer elements per
// thread per tile. 128 x 4: float32 Adam with stride-2 parameters (64 x 4M),
// same-process A/B, 4 rounds, against 128 x 8: +15% with a workspace, +12%
// without (256 x 4 +13% / +11%, 64 x 4 +10%, 128 x 16 -36%); with every
// operand at stride 2, -0.4%.
constexpr int kElemThreads = kThreads;
constexpr int kElemPer = 4;
constexpr int64_t kElemTile = int64_t(kElemThreads) * kElemPer;

// Any strides: kElemPer elements per thread, one element per access. PRE: the
// replica's constants come from the call's workspace.
template <typename P, bool PRE>
__global__ __launch_bounds__(kElemThreads) void element_kernel(KArgs<P> a) {
  using T = typename P::T;
  using S = typename P::S;
  constexpr int NS = P::NS;
  constexpr int SS = state_slots<P>();
  uint32_t r;
  int64_t t0;
  tile_of_block<kElemTile>(a.g, r, t0);
  if (!a.vec.mask[r]) {
    return;
  }
  // The workgroup's replica is every lane's: float32 Adam without a workspace
  // derives its constants once per wavefront (+4.0% on strided float32
  // parameters, same-process A/B; the segmented driver lost 1.2% with it at
  // config 5 and keeps the per-lane form).
  typename P::Rep rep;
  uniform_prologue<P, PRE>(a.vec, r, rep);
  const bool load_state = P::reads_state(a.vec, r);

  T* const prow = pg_row<P>(a.x, 0, r);
  const T* const grow = pg_row<P>(a.x, 1, r);
  S* srow[SS];
#pragma unroll
  for (int b = 0; b < NS; ++b) srow[b] = state_row<P>(a.x, 2 + b, r);
  T vp[kElemPer], vg[kElemPer];
  S vs[SS][kElemPer];
#pragma unroll
  for (int u = 0; u < kElemPer; ++u) {
    const int64_t t = t0 + int64_t(u) * kElemThreads + threadIdx.x;
    if (t < a.g.T) {
      vp[u] = prow[t * a.x.stride_t[0]];
      vg[u] = grow[t * a.x.stride_t[1]];
      if (load_state) {
#pragma unroll
        for (int b = 0; b < NS; ++b) {
          vs[b][u] = srow[b][t * a.x.stride_t[2 + b]];
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kElemPer; ++u) {
    const int64_t t = t0 + int64_t(u) * kElemThreads + threadIdx.x;
    if (t < a.g.T) {
      S st[SS];
#pragma unroll
      for (int b = 0; b < NS; ++b) st[b] = vs[b][u];
      apply_element<P>(vp[u], vg[u], st, load_state, rep, a.maximize);
      prow[t * a.x.stride_t[0]] = vp[u];
#pragma unroll
      for (int b = 0; b < NS; ++b) {
        srow[b][t * a.x.stride_t[2 + b]] = st[b];
      }
    }
  }
}

// Replica-minor operands: every (R, T) operand has unit replica stride (the
// transposed views an outer vmap over a non-leading dimension produces, or
// (T, R) buffers seen as (R, T)). A row-walking workgroup would touch one
// element per cache line there, so this driver turns the walk around: a
// workgroup covers `rb` consecutive replicas times a block of columns, each
// thread keeps one replica (its hyperparameters and per-replica constants,
// computed once) and walks columns `cpi` apart, so the threads of one
// iteration read consecutive replicas of consecutive columns -- contiguous
// memory when the column stride is R. Above 256 replicas, when 256-thread
// replica blocks would leave over a quarter of the threads idle, workgroups
// have 128 threads: R = 257 / 300 ran at 4.3 / 4.7 TB/s instead of 3.3, while
// R = 600 / 1000 / 2000 keep 256 (4.7 / 4.7 / 4.7; 128 gave 4.8 / 4.4 / 4.8).
//
// Non-temporal accesses where no cache line is shared between workgroups (one
// replica block, or replica blocks, columns and bases on 128-byte boundaries)
// and the wavefront has no frozen replica: +6-9% there (R = 8..256: 5.3 -> 5.8
// TB/s; R = 4096: 4.8 -> 5.1). Where replica blocks split lines (R = 257..2000)
// plain accesses let L2 merge the two halves: non-temporal ones ran at 2.6-3.9
// TB/s instead of 4.4-4.8. (Threads that keep four replicas and move them as
// one pack, so that a column of up to 1024 replicas has one workgroup, measured
// 0.1-0.9 TB/s slower at every R.)
constexpr int kColThreads = 256;
constexpr int kColThreadsNarrow = 128;
// Columns per thread per workgroup: 16 (config 5 as transposed views, R =
// 128, same-process A/B, two runs of 3-4 rounds: +2.2-2.6% against 32; 8:
// -1% to +2.5%, 24 and 64: -0.6% to -1.2%; against 32 at R = 64 ... 4096 on
// 2^28-element buffers: +0.7% to +1.9%).
constexpr int kColIters = 16;
constexpr int kColUnroll = 4;
constexpr uint32_t kLineBytes = 128;
constexpr uint32_t kXcds = 8;

struct ColGrid {
  int64_t R, T;
  uint32_t threads;    // workgroup size, at most kColThreads
  uint32_t rb;         // replicas per workgroup, min(R, threads)
  uint32_t cpi;        // columns per iteration, threads / rb
  uint32_t n_rblocks;  // ceil(R / rb)
};

template <typename P>
struct ColArgs {
  Operands<typename P::T> x;
  Vectors<typename P::T> vec;
  ColGrid g;
  bool maximize;
};

// One element of any storage type, plain or non-temporal.
template <typename T>
using ElemBits = std::conditional_t<sizeof(T) == 2, uint16_t,
                                    std::conditional_t<sizeof(T) == 4, uint32_t, uint64_t>>;
template <bool NT, typename T>
__device__ __forceinline__ T load_one(const T* p) {
  if constexpr (NT) {
    return __builtin_bit_cast(
        T, __builtin_nontemporal_load(reinterpret_cast<const ElemBits<T>*>(p)));
  } else {
    return *p;
  }
}
template <bool NT, typename T>
__device__ __forceinline__ void store_one(T* p, T v) {
  if constexpr (NT) {
    __builtin_nontemporal_store(__builtin_bit_cast(ElemBits<T>, v),
                                reinterpret_cast<ElemBits<T>*>(p));
  } else {
    *p = v;
  }
}

// One thread's walk over its replica's columns, plain or non-temporal.
template <typename P, bool NT>
__device__ __forceinline__ void column_walk(const ColArgs<P>& a, int64_t r, int64_t t_first,
                                            const typename P::Rep& rep, bool load_state) {
  using T = typename P::T;
  using S = typename P::S;
  constexpr int NS = P::NS;
  constexpr int SS = state_slots<P>();
  T* const pcol = a.x.data[0] + r;
  const T* const gcol = a.x.data[1] + r;
  S* scol[SS];
#pragma unroll
  for (int b = 0; b < NS; ++b) scol[b] = reinterpret_cast<S*>(a.x.data[2 + b]) + r;

  for (int j = 0; j < kColIters; j += kColUnroll) {
    T vp[kColUnroll], vg[kColUnroll];
    S vs[SS][kColUnroll];
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) {
      const int64_t t = t_first + int64_t(j + u) * a.g.cpi;
      if (t < a.g.T) {
        vp[u] = load_one<NT>(pcol + t * a.x.stride_t[0]);
        vg[u] = load_one<NT>(gcol + t * a.x.stride_t[1]);
        if (load_state) {
#pragma unroll
          for (int b = 0; b < NS; ++b) vs[b][u] = load_one<NT>(scol[b] + t * a.x.stride_t[2 + b]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) {
      const int64_t t = t_first + int64_t(j + u) * a.g.cpi;
      if (t < a.g.T) {
        S st[SS];
#pragma unroll
        for (int b = 0; b < NS; ++b) st[b] = vs[b][u];
        apply_element<P>(vp[u], vg[u], st, load_state, rep, a.maximize);
        store_one<NT>(pcol + t * a.x.stride_t[0], vp[u]);
#pragma unroll
        for (int b = 0; b < NS; ++b) store_one<NT>(scol[b] + t * a.x.stride_t[2 + b], st[b]);
      }
    }
  }
}

// NT: the launch's lines are private to workgroups (col_lines_private); a
// wavefront then goes non-temporal unless it has frozen replicas, whose
// unwritten elements would leave partial lines (non-temporal partial lines ran
// at 3.4-3.7 TB/s where plain ones ran at 4.7-4.9 with a tenth of the replicas
// frozen; non-temporal loads with plain stores were no better, 2.8-3.4).
// Storing after all four unrolled columns' arithmetic (the streaming driver's
// late stores) moved the column driver by -3% (non-temporal) to +2% (plain):
// not adopted.
// PRE: every thread reads its replica's constants from the call's workspace
// (filled by the preparation launch) instead of deriving them.
template <typename P, bool NT, bool PRE>
__global__ __launch_bounds__(kColThreads) void column_kernel(ColArgs<P> a) {
  uint32_t blk = blockIdx.x;
  if (a.g.n_rblocks > 1) {
    // The replica blocks of a column block run on one XCD: workgroups are
    // dealt to the kXcds XCDs round-robin, so XCD x takes the x-th contiguous
    // range of the remapped order, and consecutive replica blocks meet in its
    // L2 (lines split between them are fetched once). Against the plain order
    // on the same buffers: R = 257 / 300 / 1000 / 2000 4.4-4.7 -> 4.8-5.0
    // TB/s (two boxes); with private lines R = 2048 4.7 -> 5.3, R = 4096 5.0
    // -> 5.7 on one box and 5.7 -> 5.6 on another, R = 8192 5.8 either way.
    // With one replica block the plain order is faster (R <= 256: 5.8 against
    // 5.0-5.5 remapped).
    const uint32_t n = gridDim.x, x = blockIdx.x % kXcds, per = n / kXcds, rem = n % kXcds;
    blk = x * per + (x < rem ? x : rem) + blockIdx.x / kXcds;
  }
  const uint32_t rblk = blk % a.g.n_rblocks;
  const uint32_t cblk = blk / a.g.n_rblocks;
  const uint32_t rr = threadIdx.x % a.g.rb;
  const uint32_t cc = threadIdx.x / a.g.rb;
  const int64_t r = int64_t(rblk) * a.g.rb + rr;
  const bool in_range = cc < a.g.cpi && r < a.g.R;
  const bool active = in_range && a.vec.mask[r];
  bool nt = false;
  if constexpr (NT) {
    nt = __ballot(in_range) == __ballot(active);
  }
  // Threads past the last replica or column lane, and frozen replicas, have
  // nothing to do (the workgroup has no barrier).
  if (!active) {
    return;
  }
  typename P::Rep rep;
  P::template prologue<PRE>(a.vec, static_cast<uint32_t>(r), rep);
  const bool load_state = P::reads_state(a.vec, static_cast<uint32_t>(r));
  const int64_t t_first = int64_t(cblk) * a.g.cpi * kColIters + cc;
  if (nt) {
    column_walk<P, true>(a, r, t_first, rep, load_state);
  } else {
    column_walk<P, false>(a, r, t_first, rep, load_state);
  }
}

// ---------------------------------------------------------------------------
// Segmented gradients
// ---------------------------------------------------------------------------
constexpr int kMaxSegments = 64;

// Up to kMaxSegments per-parameter (R, numel) tensors, each mapped onto the
// columns [col, col + numel) of the (R, T) layout. tile0 is the prefix sum of
// the segments' tile counts, so a row has tile0[n] tiles; bit s of `vec_ok`
// says segment s takes the vector walk (the (R, T) operands are streamable and
// the segment's data is element-aligned).
template <typename T>
struct Segments {
  const T* data[kMaxSegments];
  int64_t stride_r[kMaxSegments];
  int64_t col[kMaxSegments];
  int64_t numel[kMaxSegments];
  uint32_t tile0[kMaxSegments + 1];
  uint64_t vec_ok;
  int n;
};

template <typename P>
struct SegArgs {
  KArgs<P> k;  // k.x.data[1]: consolidated gradient to write, or null;
               // k.g.res0 / rmod: the params rows' phase
  Segments<typename P::T> seg;
};

__device__ __forceinline__ int segment_of_tile(const uint32_t* tile0, int n, uint32_t t) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tile0[mid] <= t) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// A segment's tile on the vector walk. The walk follows the (R, T) layout: in
// row r the segment's first 256-byte boundary lies `head` elements in (head <
// A, as for the streaming driver); packs of 4 elements stream from there, tile
// k taking packs [k * TILE / 4, (k + 1) * TILE / 4). Tile 0 also takes the
// head elements and the segment's last tile the at most three tail elements,
// one element per access. The per-parameter gradient's rows keep their own
// alignment: they are read with element-aligned pack loads.
struct SegTile {
  int64_t head;   // elements before the first pack
  int64_t first;  // element index of this tile's first pack
  int64_t packs;  // packs in this tile (may be <= 0)
  int64_t tail;   // first tail element (== numel: none)
  bool has_head, has_tail;
};

template <typename T, int64_t TILE, int KP>
__device__ __forceinline__ SegTile seg_tile(uint32_t res0, uint32_t rmod, uint32_t r,
                                            int64_t col, int64_t numel, int64_t j0) {
  constexpr uint32_t A = align_elems<T>();
  SegTile t;
  const uint32_t phase = (res0 + r * rmod + static_cast<uint32_t>(col % A)) % A;
  t.head = imin(numel, (A - phase) % A);
  const int64_t packs_seg = (numel - t.head) / KP;
  t.first = t.head + j0;
  t.packs = packs_seg - j0 / KP;
  t.tail = t.head + packs_seg * KP;
  t.has_head = j0 == 0;
  t.has_tail = j0 + TILE >= numel;
  return t;
}

// Runs fn(j) for the tile's single elements, spread over the NTH threads.
template <int NTH, typename Fn>
__device__ __forceinline__ void seg_singles(const SegTile& t, int64_t numel, Fn&& fn) {
  if (t.has_head) {
    for (int64_t j = threadIdx.x; j < t.head; j += NTH) fn(j);
  }
  if (t.has_tail) {
    for (int64_t j = t.tail + threadIdx.x; j < numel; j += NTH) fn(j);
  }
}

// PRE: the per-replica constants come from the call's workspace (a.k.vec.pre).
template <typename P, bool ANY, bool PRE>
__global__ __launch_bounds__((segment_threads<P, PRE>())) void segment_kernel(SegArgs<P> a) {
  using T = typename P::T;
  using S = typename P::S;
  constexpr int NS = P::NS;
  constexpr int SS = state_slots<P>();
  constexpr int U = segment_unroll<P, PRE>();
  constexpr int NTH = segment_threads<P, PRE>();
  constexpr int64_t kSegTile = segment_tile<P, PRE>();
  // 16 B per lane and access, as in the streaming driver (4-element packs had
  // given 16-bit operands 8 B per lane and float64 32 B, two accesses over
  // every other 16 B: float64 +16% for Adam and SGD with 16-byte packs, 16-bit
  // within -1.3% to +4% at half the packs per thread; same-process A/B on
  // config 5's per-parameter gradients).
  constexpr int KP = stream_pack<T, S>();
  const uint32_t tiles_per_row = a.seg.tile0[a.seg.n];
  const uint32_t r = blockIdx.x / tiles_per_row;
  const uint32_t local = blockIdx.x - r * tiles_per_row;
  const bool write_grad = a.k.x.data[1] != nullptr;
  const bool active = segment_scalar_mask_of<P>::value ? mask_byte_scalar(a.k.vec.mask, r)
                                                        : a.k.vec.mask[r] != 0;
  const int s = segment_of_tile(a.seg.tile0, a.seg.n, local);
  // A segment without data is a gap between gradients: its columns take the
  // gradient already in the consolidated buffer, or zero when there is none.
  const bool gap = a.seg.data[s] == nullptr;
  if (!active && (gap || !write_grad)) {
    return;
  }
  const int64_t numel = a.seg.numel[s];
  const int64_t col = a.seg.col[s];
  const int64_t j0 = int64_t(local - a.seg.tile0[s]) * kSegTile;
  const bool vec = (a.seg.vec_ok >> s) & 1u;
  // Row r of the segment's columns in the (R, T) operands, and of its gradient
  // source: the segment's row, or for a gap the consolidated buffer (null:
  // zero). Only a real segment is stored into the consolidated buffer.
  T* const g_dst =
      write_grad ? pg_row<P>(a.k.x, 1, r) + col * a.k.x.stride_t[1] : nullptr;
  const T* g_src = g_dst;
  int64_t g_stride = write_grad ? a.k.x.stride_t[1] : 0;
  if (!gap) {
    g_src = a.seg.data[s] + int64_t(r) * a.seg.stride_r[s];
    g_stride = 1;
  }
  const bool store_grad = write_grad && !gap;

  if (!active) {
    // A frozen replica's optimizer state is not touched, but the consolidated
    // gradient is still filled, as the separate scatter would have filled it.
    if (vec) {
      const SegTile t = seg_tile<T, kSegTile, KP>(a.k.g.res0, a.k.g.rmod, r, col, numel, j0);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = int64_t(u) * NTH + threadIdx.x;
        if (i < t.packs) {
          Packs<ANY, T, true, KP>(g_dst + t.first)
              .store(i, load_stream_any<true, KP>(g_src + t.first + i * KP));
        }
      }
      seg_singles<NTH>(t, numel, [&](int64_t j) { g_dst[j] = g_src[j]; });
    } else {
      const int64_t cnt = imin(kSegTile, numel - j0);
      for (int64_t j = j0 + threadIdx.x; j < j0 + cnt; j += NTH) {
        g_dst[j * a.k.x.stride_t[1]] = g_src[j];
      }
    }
    return;
  }

  typename P::Rep rep;
  P::template prologue<PRE>(a.k.vec, r, rep);
  const bool load_state = P::reads_state(a.k.vec, r);
  const T zero = narrow<T>(op_t<T>(0));

  T* const prow = pg_row<P>(a.k.x, 0, r) + col * a.k.x.stride_t[0];
  S* srow[SS];
#pragma unroll
  for (int b = 0; b < NS; ++b) {
    srow[b] = state_row<P>(a.k.x, 2 + b, r) + col * a.k.x.stride_t[2 + b];
  }

  // Element j of the segment, one access per operand.
  const auto one = [&](int64_t j) {
    T p = prow[j * a.k.x.stride_t[0]];
    const T g = g_src != nullptr ? g_src[j * g_stride] : zero;
    S st[SS];
    if (load_state) {
#pragma unroll
      for (int b = 0; b < NS; ++b) st[b] = srow[b][j * a.k.x.stride_t[2 + b]];
    }
    apply_element<P>(p, g, st, load_state, rep, a.k.maximize);
    prow[j * a.k.x.stride_t[0]] = p;
    if (store_grad) {
      g_dst[j * a.k.x.stride_t[1]] = g;
    }
#pragma unroll
    for (int b = 0; b < NS; ++b) srow[b][j * a.k.x.stride_t[2 + b]] = st[b];
  };

  if (!vec) {
    const int64_t cnt = imin(kSegTile, numel - j0);
    for (int64_t j = j0 + threadIdx.x; j < j0 + cnt; j += NTH) one(j);
    return;
  }

  // Vector walk (unit inner strides): the parameters' packs are aligned; with
  // ANY the other operands sit at another 16-byte phase (element-aligned packs).
  const SegTile t = seg_tile<T, kSegTile, KP>(a.k.g.res0, a.k.g.rmod, r, col, numel, j0);
  Pack<T, KP>* const pp = reinterpret_cast<Pack<T, KP>*>(prow + t.first);
  Packs<ANY, S, true, KP> sp[SS];
#pragma unroll
  for (int b = 0; b < NS; ++b) sp[b] = Packs<ANY, S, true, KP>(srow[b] + t.first);
  const Packs<ANY, T, true, KP> gout(g_dst != nullptr ? g_dst + t.first : nullptr);
  Pack<T, KP> vp[U], vg[U];
  Pack<S, KP> vs[SS][U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = int64_t(u) * NTH + threadIdx.x;
    if (i < t.packs) {
      vp[u] = load_stream(pp + i);
      if (gap) {
        if (g_src != nullptr) {
          vg[u] = gout.load(i);  // a gap reads the consolidated gradient
        } else {
#pragma unroll
          for (int k = 0; k < KP; ++k) vg[u].v[k] = zero;
        }
      } else {
        vg[u] = load_stream_any<true, KP>(g_src + t.first + i * KP);
      }
      if (load_state) {
#pragma unroll
        for (int b = 0; b < NS; ++b) vs[b][u] = sp[b].load(i);
      }
    }
  }
  with_variant<P>(rep, [&](const typename P::Rep& rp) {
    with_maximize<P>(a.k.maximize, [&](bool mx) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = int64_t(u) * NTH + threadIdx.x;
        if (i < t.packs) {
          if (store_grad) {
            gout.store(i, vg[u]);
          }
          Pack<S, KP> st[SS];
#pragma unroll
          for (int b = 0; b < NS; ++b) st[b] = vs[b][u];
          apply_pack<P, KP>(vp[u], vg[u], st, load_state, rp, mx);
#pragma unroll
          for (int b = 0; b < NS; ++b) vs[b][u] = st[b];
          store_stream(pp + i, vp[u]);
#pragma unroll
          for (int b = 0; b < NS; ++b) sp[b].store(i, vs[b][u]);
        }
      }
    });
  });
  seg_singles<NTH>(t, numel, one);
}

// Plain gradient scatter: copies every segment into its columns of the (R, T)
// destination, every row (frozen replicas included, as a copy would). The
// vector walk follows the destination's 256-byte boundaries (res0 / rmod as
// for the update).
template <typename T>
struct ScatterArgs {
  T* dst;
  int64_t dst_stride_r;
  uint32_t res0, rmod;
  Segments<T> seg;
};

// The scatter's workgroup shape: kScatterThreads threads x kScatterUnroll
// packs of 4 elements per tile, under a residency cap of kScatterLds bytes of
// dynamic LDS (0: none). Same-process A/B on config 5's twelve per-parameter
// gradients (23.6 GB moved, 4 rounds): one wavefront x 1 pack 6.71 TB/s;
// 128 x 2 6.48, 256 x 1 6.54, 128 x 1 6.44, 64 x 4 6.29, 64 x 2 5.95; caps of
// 12-16 workgroups per CU 4.7-4.9.
constexpr int kScatterThreads = 64;
constexpr int kScatterUnroll = 1;
constexpr uint32_t kScatterLds = 0;
// Elements per pack of the scatter: 16 B per lane and access (config 5's
// layout, same-process A/B against 4-element packs: float16 3.87 -> 6.71
// TB/s, float64 3.30 -> 6.72).
template <typename T>
constexpr int scatter_pack() {
  return static_cast<int>(16 / sizeof(T));
}
template <typename T>
constexpr int64_t scatter_tile() {
  return int64_t(kScatterThreads) * scatter_pack<T>() * kScatterUnroll;
}

template <typename T>
__global__ __launch_bounds__(kScatterThreads) void scatter_kernel(ScatterArgs<T> a) {
  constexpr int KP = scatter_pack<T>();
  constexpr int64_t kScatterTile = scatter_tile<T>();
  const uint32_t tiles_per_row = a.seg.tile0[a.seg.n];
  const uint32_t r = blockIdx.x / tiles_per_row;
  const uint32_t local = blockIdx.x - r * tiles_per_row;
  const int s = segment_of_tile(a.seg.tile0, a.seg.n, local);
  const int64_t numel = a.seg.numel[s];
  const int64_t j0 = int64_t(local - a.seg.tile0[s]) * kScatterTile;
  const T* src = a.seg.data[s] + int64_t(r) * a.seg.stride_r[s];
  T* dst = a.dst + int64_t(r) * a.dst_stride_r + a.seg.col[s];
  if ((a.seg.vec_ok >> s) & 1u) {
    const SegTile t = seg_tile<T, kScatterTile, KP>(a.res0, a.rmod, r, a.seg.col[s], numel, j0);
    Pack<T, KP> v[kScatterUnroll];
#pragma unroll
    for (int u = 0; u < kScatterUnroll; ++u) {
      const int64_t i = int64_t(u) * kScatterThreads + threadIdx.x;
      if (i < t.packs) v[u] = load_stream_any<true, KP>(src + t.first + i * KP);
    }
#pragma unroll
    for (int u = 0; u < kScatterUnroll; ++u) {
      const int64_t i = int64_t(u) * kScatterThreads + threadIdx.x;
      if (i < t.packs) store_stream(reinterpret_cast<Pack<T, KP>*>(dst + t.first) + i, v[u]);
    }
    seg_singles<kScatterThreads>(t, numel, [&](int64_t j) { dst[j] = src[j]; });
    return;
  }
  const int64_t cnt = imin(kScatterTile, numel - j0);
  for (int64_t j = j0 + threadIdx.x; j < j0 + cnt; j += kScatterThreads) {
    dst[j] = src[j];
  }
}

// ---------------------------------------------------------------------------
// state_steps += active_mask, and the zero return scalar.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kThreads) void bump_steps_kernel(
    T* __restrict__ steps, const uint8_t* __restrict__ mask, int64_t R,
    T* __restrict__ out_zero) {
  const int64_t r = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (r < R) {
    const op_t<T> one = mask[r] ? op_t<T>(1) : op_t<T>(0);
    steps[r] = narrow<T>(widen(steps[r]) + one);
  }
  if (out_zero != nullptr && r == 0) {
    *out_zero = narrow<T>(op_t<T>(0));
  }
}

// The preparation launch of a call with a workspace: the optional step bump
// (as bump_steps_kernel), then each active replica's constants from the
// stored, bumped step into pre + kPreStride * r (frozen replicas' entries are
// neither written nor read), and the zero result. `v.steps` points at `steps`.
template <typename P>
__global__ __launch_bounds__(kThreads) void prep_kernel(Vectors<typename P::T> v,
                                                        typename P::T* steps, int64_t R,
                                                        bool bump, double* pre,
                                                        typename P::T* out_zero) {
  using T = typename P::T;
  const int64_t r = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (r < R) {
    const bool active = v.mask[r] != 0;
    if (bump) {
      const op_t<T> one = active ? op_t<T>(1) : op_t<T>(0);
      steps[r] = narrow<T>(widen(steps[r]) + one);
    }
    if (active) {
      P::precompute(v, static_cast<uint32_t>(r), pre + kPreStride * r);
    }
  }
  if (out_zero != nullptr && r == 0) {
    *out_zero = narrow<T>(op_t<T>(0));
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr int kInvalid = static_cast<int>(hipErrorInvalidValue);

template <typename T>
bool fill_operands(const ts_rt_buf* bufs, int n, Operands<T>& x, bool grad_optional) {
  for (int b = 0; b < kMaxOperands; ++b) {
    x.data[b] = nullptr;
    x.stride_r[b] = 0;
    x.stride_t[b] = 1;
  }
  for (int b = 0; b < n; ++b) {
    if (bufs[b].data == nullptr) {
      if (b == 1 && grad_optional) continue;
      return false;
    }
    x.data[b] = static_cast<T*>(bufs[b].data);
    x.stride_r[b] = bufs[b].stride_r;
    x.stride_t[b] = bufs[b].stride_t;
  }
  return true;
}

// The streaming drivers take any operands with unit inner stride and
// element-aligned bases. The walk follows the parameters' boundaries (res0 /
// rmod: their phase modulo kPhaseBytes, for the grid); operands at another
// phase use element-aligned packs.
template <typename P>
bool rows_streamable(const Operands<typename P::T>& x, int n, uint32_t& res0, uint32_t& rmod) {
  constexpr uint32_t A = phase_elems<typename P::T>();
  for (int b = 0; b < n; ++b) {
    if (x.data[b] == nullptr) continue;
    const size_t elem = b < 2 ? sizeof(typename P::T) : sizeof(typename P::S);
    const uintptr_t addr = reinterpret_cast<uintptr_t>(x.data[b]);
    if (x.stride_t[b] != 1 || addr % elem != 0) return false;
  }
  const uintptr_t p0 = reinterpret_cast<uintptr_t>(x.data[0]);
  res0 = static_cast<uint32_t>((p0 / sizeof(typename P::T)) % A);
  rmod = static_cast<uint32_t>(((x.stride_r[0] % A) + A) % A);
  return true;
}

// Whether every present operand's pack boundaries (packs of `pack` elements)
// fall on the same element index as the parameters' in every row (common base
// residue and row stride modulo `pack`): then all packs are aligned and the
// drivers' ANY = false variants run.
template <typename P>
bool rows_same_phase(const Operands<typename P::T>& x, int n, int64_t pack = kPack) {
  const auto residue = [&](int b) {
    const size_t elem = b < 2 ? sizeof(typename P::T) : sizeof(typename P::S);
    return static_cast<uint32_t>((reinterpret_cast<uintptr_t>(x.data[b]) / elem) % pack);
  };
  const auto mod = [&](int b) {
    return static_cast<uint32_t>(((x.stride_r[b] % pack) + pack) % pack);
  };
  for (int b = 1; b < n; ++b) {
    if (x.data[b] == nullptr) continue;
    if (residue(b) != residue(0) || mod(b) != mod(0)) return false;
  }
  return true;
}

// Every present operand has unit replica stride (and R > 1, where that says
// anything): the column driver's layout.
template <typename T>
bool replica_minor(const Operands<T>& x, int n) {
  for (int b = 0; b < n; ++b) {
    if (x.data[b] != nullptr && x.stride_r[b] != 1) return false;
  }
  return true;
}

// Whether a 1-D grid of `blocks` workgroups of `threads` threads can launch:
// at most INT32_MAX workgroups, and at most 2^32 - 1 work-items (the dispatch
// packet counts work-items in 32 bits; HIP refuses a larger launch, which would
// leave a call's preparation launch run and its update not).
inline bool grid_fits(uint64_t blocks, int threads) {
  return blocks <= INT32_MAX && blocks * static_cast<uint64_t>(threads) <= UINT32_MAX;
}

inline bool make_col_grid(int64_t R, int64_t T, ColGrid& g, uint32_t& blocks) {
  if (R <= 1 || R > INT32_MAX || T <= 0) return false;
  g.R = R;
  g.T = T;
  g.threads = kColThreads;
  if (R > kColThreads) {
    // 256-thread replica blocks that would leave over a quarter of their
    // threads idle (R = 257..341, 513..682, ...) give way to 128.
    const int64_t span = (R + kColThreads - 1) / kColThreads * kColThreads;
    if (4 * (span - R) > span) g.threads = kColThreadsNarrow;
  }
  g.rb = static_cast<uint32_t>(std::min<int64_t>(R, g.threads));
  g.cpi = g.threads / g.rb;
  const int64_t n_rblocks = (R + g.rb - 1) / g.rb;
  const int64_t cols_per_block = int64_t(g.cpi) * kColIters;
  const int64_t n_cblocks = (T + cols_per_block - 1) / cols_per_block;
  if (n_rblocks > INT32_MAX / n_cblocks ||
      !grid_fits(static_cast<uint64_t>(n_rblocks * n_cblocks), g.threads)) {
    return false;  // the element driver takes it
  }
  g.n_rblocks = static_cast<uint32_t>(n_rblocks);
  blocks = static_cast<uint32_t>(n_rblocks * n_cblocks);
  return true;
}

// No cache line of the column driver's operands is shared between two
// workgroups: one replica block per column, or replica blocks, columns and
// bases all on 128-byte boundaries.
template <typename P>
bool col_lines_private(const Operands<typename P::T>& x, int n, const ColGrid& g) {
  if (g.n_rblocks == 1) return true;
  for (int b = 0; b < n; ++b) {
    if (x.data[b] == nullptr) continue;
    const size_t es = b < 2 ? sizeof(typename P::T) : sizeof(typename P::S);
    if (reinterpret_cast<uintptr_t>(x.data[b]) % kLineBytes != 0 ||
        uint64_t(x.stride_t[b]) * es % kLineBytes != 0 || g.rb * es % kLineBytes != 0) {
      return false;
    }
  }
  return true;
}

// The (replica, tile) grid of a row driver, in `threads`-thread workgroups.
// With head_tiles (the streaming driver) every row also gets its tile 0, the
// first R workgroups; its ceil(T / tile) other tiles cover
// [head, head + ceil(T / tile) * tile) ⊇ [head, T), the last of them empty
// where the head and the tail fit in one.
inline bool make_grid(int64_t R, int64_t T, int64_t tile, Grid& g, uint32_t& blocks,
                      int threads, bool head_tiles = false) {
  const int64_t tiles = (T + tile - 1) / tile + (head_tiles ? 1 : 0);
  if (R <= 0 || T <= 0 || tiles > INT32_MAX || R > INT32_MAX / tiles ||
      !grid_fits(static_cast<uint64_t>(R) * static_cast<uint64_t>(tiles), threads)) {
    return false;
  }
  g.T = T;
  g.tiles_per_row = static_cast<uint32_t>(head_tiles ? tiles - 1 : tiles);
  set_div_tiles(g);
  g.res0 = 0;
  g.rmod = 0;
  g.heads = head_tiles ? static_cast<uint32_t>(R) : 0u;
  blocks = static_cast<uint32_t>(R * tiles);
  return true;
}

template <typename T>
int launch_bump(void* steps, const uint8_t* mask, int64_t R, void* out_zero,
                hipStream_t stream) {
  const int64_t blocks = R > 0 ? (R + kThreads - 1) / kThreads : 1;
  if (blocks > INT32_MAX) {
    return kInvalid;
  }
  hipLaunchKernelGGL(bump_steps_kernel<T>, dim3(static_cast<uint32_t>(blocks)),
                     dim3(kThreads), 0, stream, static_cast<T*>(steps), mask, R,
                     static_cast<T*>(out_zero));
  return static_cast<int>(hipGetLastError());
}

// A caller's segment table: in column order, disjoint, inside [0, cols), with
// data for every non-empty segment (two tiles writing one column would race).
// One pass, no allocation.
inline bool segments_valid(const ts_segment* segs, int n, int64_t cols) {
  int64_t end = 0;
  for (int i = 0; i < n; ++i) {
    const ts_segment& s = segs[i];
    if (s.numel < 0 || s.col < 0 || s.col > cols - s.numel) return false;
    if (s.numel == 0) continue;
    if (s.data == nullptr || s.col < end) return false;
    end = s.col + s.numel;
  }
  return true;
}

// Walks a valid table in column order, skipping empty segments. With `gaps`,
// the column ranges no segment covers (between segments and after the last
// one, up to `cols`) come out as entries without data.
struct SegmentWalk {
  const ts_segment* segs;
  int n;
  int64_t cols;
  bool gaps;
  int i = 0;
  int64_t at = 0;

  bool next(ts_segment& out) {
    while (i < n && segs[i].numel == 0) ++i;
    const int64_t stop = i < n ? segs[i].col : cols;
    if (gaps && at < stop) {
      out = ts_segment{nullptr, 0, at, stop - at};
      at = stop;
      return true;
    }
    if (i == n) return false;
    out = segs[i++];
    at = out.col + out.numel;
    return true;
  }
};

// Fills the next launch's table, up to kMaxSegments entries, from the walk;
// returns the grid size (0 when the walk is done, -1 when it exceeds the 1-D
// grid of `threads`-thread workgroups). `vec_rows` says whether the (R, T)
// operands allow vector access.
template <typename T>
int64_t next_chunk(SegmentWalk& w, int64_t R, int64_t tile, bool vec_rows, Segments<T>& out,
                   int threads) {
  out.n = 0;
  out.vec_ok = 0;
  uint64_t tiles = 0;
  ts_segment s;
  while (out.n < kMaxSegments && w.next(s)) {
    const int k = out.n++;
    out.data[k] = static_cast<const T*>(s.data);
    out.stride_r[k] = s.stride_r;
    out.col[k] = s.col;
    out.numel[k] = s.numel;
    out.tile0[k] = static_cast<uint32_t>(tiles);
    tiles += static_cast<uint64_t>((s.numel + tile - 1) / tile);
    if (tiles > UINT32_MAX) return -1;
    const bool ok = vec_rows && reinterpret_cast<uintptr_t>(s.data) % sizeof(T) == 0;
    out.vec_ok |= (ok ? uint64_t(1) : uint64_t(0)) << k;
  }
  out.tile0[out.n] = static_cast<uint32_t>(tiles);
  const uint64_t blocks = tiles * static_cast<uint64_t>(R);
  return grid_fits(blocks, threads) ? static_cast<int64_t>(blocks) : -1;
}

// Checks that every launch of a walk fits the grid, without launching.
template <typename T>
bool walk_fits(SegmentWalk w, int64_t R, int64_t tile, bool vec_rows, Segments<T>& scratch,
               int threads = kThreads) {
  int64_t blocks;
  while ((blocks = next_chunk<T>(w, R, tile, vec_rows, scratch, threads)) != 0 || scratch.n > 0) {
    if (blocks < 0) return false;
  }
  return true;
}

// Launches `kernel` once per chunk of the walk.
template <typename T, typename Args, typename Kernel>
int launch_walk(SegmentWalk w, int64_t R, int64_t tile, bool vec_rows, Args& a, Segments<T>& seg,
                Kernel kernel, hipStream_t stream, uint32_t lds = 0, int threads = kThreads) {
  int64_t blocks;
  while ((blocks = next_chunk<T>(w, R, tile, vec_rows, seg, threads)) != 0 || seg.n > 0) {
    if (blocks < 0) return kInvalid;
    if (blocks == 0) continue;
    hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(blocks)), dim3(threads), lds, stream,
                       a);
    const int err = static_cast<int>(hipGetLastError());
    if (err != 0) return err;
  }
  return 0;
}

// A call: the (R, T) operand table, the (R,) vectors, the flags and the
// optional workspace for per-replica constants.
struct Call {
  const ts_rt_buf* bufs;
  void* steps;
  const void* h[5];
  int nh;
  const uint8_t* mask;
  int64_t R, T;
  uint32_t flags;
  void* out_zero;
  void* ws;
  size_t ws_bytes;
  hipStream_t stream;
};

// Whether policy P takes its per-replica constants from the call's workspace.
template <typename P>
bool uses_workspace(const Call& c) {
  return P::kPreWords > 0 && c.ws != nullptr;
}

// The rule ilp_row decodes, over the first three operands (parameters,
// gradients, first state; an absent gradient counts as aligned, as the
// freshly allocated buffer it stands for).
template <typename P>
uint32_t ilp_rows_rule(const Operands<typename P::T>& x, int64_t cols) {
  if (cols % 4 != 0) return 0;
  uint32_t rule = 1;
  for (int b = 0; b < 3; ++b) {
    if (x.data[b] == nullptr) continue;
    const size_t elem = b < 2 ? sizeof(typename P::T) : sizeof(typename P::S);
    const uintptr_t addr = reinterpret_cast<uintptr_t>(x.data[b]);
    if (x.stride_t[b] != 1 || addr % elem != 0) return 0;
    const uint32_t res = static_cast<uint32_t>((addr / elem) % 4);
    const uint32_t mod = static_cast<uint32_t>(((x.stride_r[b] % 4) + 4) % 4);
    rule |= res << (1 + 4 * b) | mod << (3 + 4 * b);
  }
  return rule;
}

template <typename P>
bool fill_kargs(const Call& c, int nbufs, KArgs<P>& a, bool grad_optional) {
  using T = typename P::T;
  if (!fill_operands<T>(c.bufs, nbufs, a.x, grad_optional)) return false;
  a.vec.steps = static_cast<const T*>(c.steps);
  for (int i = 0; i < 5; ++i) {
    a.vec.h[i] = i < c.nh ? static_cast<const T*>(c.h[i]) : nullptr;
    if (i < c.nh && c.h[i] == nullptr) return false;
  }
  a.vec.mask = c.mask;
  a.vec.pre = uses_workspace<P>(c) ? static_cast<const double*>(c.ws) : nullptr;
  a.vec.ilp_rows = ilp_rows_rule<P>(a.x, c.T);
  a.maximize = (c.flags & TS_MAXIMIZE) != 0;
  return true;
}

template <typename P>
int launch_prep(const Call& c, const Vectors<typename P::T>& vec) {
  using T = typename P::T;
  const int64_t blocks = (c.R + kThreads - 1) / kThreads;
  if (blocks > INT32_MAX) {
    return kInvalid;
  }
  hipLaunchKernelGGL(prep_kernel<P>, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                     c.stream, vec, static_cast<T*>(c.steps), c.R,
                     (c.flags & TS_BUMP_STEPS) != 0, static_cast<double*>(c.ws),
                     static_cast<T*>(c.out_zero));
  return static_cast<int>(hipGetLastError());
}

// Validation, then the preparation launch (the optional bump and the zero
// result; with a workspace also the per-replica constants), then `launch`
// when there is any work. Every check happens before the first enqueue, so an
// invalid call changes nothing. Empty tensors may carry null data pointers, so
// operands are only required where they are dereferenced: steps and mask when
// R > 0, the rest (checked by `prepare`, which also fills the kernel arguments
// in `vec`) when there is at least one element. A workspace must hold
// kPreStride doubles per replica and be 8-byte aligned.
template <typename P, typename Prepare, typename Launch>
int run_step(const Call& c, const Vectors<typename P::T>& vec, Prepare&& prepare,
             Launch&& launch) {
  using T = typename P::T;
  if (c.bufs == nullptr || c.R < 0 || c.T < 0 ||
      (c.R > 0 && (c.steps == nullptr || c.mask == nullptr))) {
    return kInvalid;
  }
  if (c.ws != nullptr &&
      (reinterpret_cast<uintptr_t>(c.ws) % alignof(double) != 0 ||
       c.ws_bytes / (kPreStride * sizeof(double)) < static_cast<uint64_t>(c.R))) {
    return kInvalid;
  }
  const bool work = c.R > 0 && c.T > 0;
  if (work && !prepare()) {
    return kInvalid;
  }
  if (work && uses_workspace<P>(c)) {
    const int err = launch_prep<P>(c, vec);
    if (err != 0) return err;
  } else if ((c.flags & TS_BUMP_STEPS) != 0 && c.R > 0) {
    const int err = launch_bump<T>(c.steps, c.mask, c.R, c.out_zero, c.stream);
    if (err != 0) return err;
  } else if (c.out_zero != nullptr) {
    const int err = launch_bump<T>(c.steps, c.mask, 0, c.out_zero, c.stream);
    if (err != 0) return err;
  }
  if (!work) {
    return 0;
  }
  return launch();
}

// The column driver over `blocks` workgroups: non-temporal when no cache line
// is shared between workgroups; PRE with the call's workspace.
template <typename P, bool PRE>
void launch_column(const ColArgs<P>& ca, uint32_t blocks, bool private_lines,
                   hipStream_t stream) {
  if (private_lines) {
    hipLaunchKernelGGL((column_kernel<P, true, PRE>), dim3(blocks), dim3(ca.g.threads), 0, stream,
                       ca);
  } else {
    hipLaunchKernelGGL((column_kernel<P, false, PRE>), dim3(blocks), dim3(ca.g.threads), 0,
                       stream, ca);
  }
}

// The streaming driver over `blocks` tiles, capped when the launch is large
// (`mid`: the operands take at most kMidBytes; with a workspace only).
template <typename P, bool PRE, bool SMALL>
void launch_stream(const KArgs<P>& a, uint32_t blocks, bool same_phase, hipStream_t stream,
                   bool mid = false) {
  const uint32_t cap = PRE && !SMALL && mid ? P::kStreamLdsMid : stream_lds_of<P, PRE, SMALL>();
  const uint32_t lds = int64_t(blocks) * stream_tile<P, PRE, SMALL>() >= kCapMinElems ? cap : 0u;
  if (same_phase) {
    hipLaunchKernelGGL((stream_kernel<P, false, PRE, SMALL>), dim3(blocks),
                       dim3(stream_threads<P, SMALL>()), lds, stream, a);
  } else {
    hipLaunchKernelGGL((stream_kernel<P, true, PRE, SMALL>), dim3(blocks),
                       dim3(stream_threads<P, SMALL>()), lds, stream, a);
  }
}

// Consolidated-gradient update with policy P over `nbufs` operands.
template <typename P>
int launch_dense(const Call& c, int nbufs) {
  KArgs<P> a;
  uint32_t blocks = 0;
  bool streamable = false;
  const bool pre = uses_workspace<P>(c);
  // Operands that fit the MALL (R, T and the types say so, before any launch).
  // The small shape is built for the forms the operators run: with a
  // workspace where the policy has one, and for SGD, which has none.
  const bool small =
      (pre || P::kPreWords == 0) &&
      c.R <= P::kStreamSmallBytes / operand_bytes_per_elem<P>() / std::max<int64_t>(c.T, 1);
  const bool mid =
      c.R <= kMidBytes / operand_bytes_per_elem<P>() / std::max<int64_t>(c.T, 1);
  const auto prepare = [&] {
    if (!fill_kargs<P>(c, nbufs, a, false)) return false;
    uint32_t res0 = 0, rmod = 0;
    streamable = rows_streamable<P>(a.x, nbufs, res0, rmod);
    const int64_t tile = !streamable ? kElemTile
                         : small     ? stream_tile<P, false, true>()
                         : pre       ? stream_tile<P, true, false>()
                                     : stream_tile<P, false, false>();
    const int threads = !streamable ? kElemThreads
                        : small     ? stream_threads<P, true>()
                                    : stream_threads<P, false>();
    // The streaming driver adds each row's tile 0 (its head and tail).
    if (!make_grid(c.R, c.T, tile, a.g, blocks, threads, streamable)) return false;
    a.g.res0 = res0;
    a.g.rmod = rmod;
    return true;
  };
  return run_step<P>(c, a.vec, prepare, [&]() -> int {
    const dim3 grid(blocks), block(kElemThreads);
    ColArgs<P> ca;
    uint32_t col_blocks = 0;
    if (streamable) {
      const bool same_phase = rows_same_phase<P>(a.x, nbufs, P::kStreamPack);
      if constexpr (P::kPreWords > 0) {
        if (pre) {
          if (small) {
            launch_stream<P, true, true>(a, blocks, same_phase, c.stream);
          } else {
            launch_stream<P, true, false>(a, blocks, same_phase, c.stream, mid);
          }
          return static_cast<int>(hipGetLastError());
        }
      }
      if constexpr (P::kPreWords == 0) {
        if (small) {
          launch_stream<P, false, true>(a, blocks, same_phase, c.stream);
          return static_cast<int>(hipGetLastError());
        }
      }
      launch_stream<P, false, false>(a, blocks, same_phase, c.stream);
    } else if (replica_minor(a.x, nbufs) && make_col_grid(c.R, c.T, ca.g, col_blocks)) {
      ca.x = a.x;
      ca.vec = a.vec;
      ca.maximize = a.maximize;
      const bool private_lines = col_lines_private<P>(a.x, nbufs, ca.g);
      if constexpr (P::kPreWords > 0) {
        if (pre) {
          launch_column<P, true>(ca, col_blocks, private_lines, c.stream);
          return static_cast<int>(hipGetLastError());
        }
      }
      launch_column<P, false>(ca, col_blocks, private_lines, c.stream);
    } else {
      if constexpr (P::kPreWords > 0) {
        if (pre) {
          hipLaunchKernelGGL((element_kernel<P, true>), grid, block, 0, c.stream, a);
          return static_cast<int>(hipGetLastError());
        }
      }
      hipLaunchKernelGGL((element_kernel<P, false>), grid, block, 0, c.stream, a);
    }
    return static_cast<int>(hipGetLastError());
  });
}

// Segmented-gradient update with policy P: one launch per kMaxSegments
// entries of the walk (their columns are disjoint, so the launches are
// independent). The gaps make the result that of a scatter followed by the
// consolidated update in every column.
template <typename P>
int launch_segments(const Call& c, int nbufs, const ts_segment* segs, int n_segs) {
  using T = typename P::T;
  if (n_segs < 0 || (n_segs > 0 && segs == nullptr)) return kInvalid;
  SegArgs<P> a;
  bool vec_rows = false;
  const SegmentWalk walk{segs, n_segs, c.T, true};
  const bool pre = uses_workspace<P>(c);
  const int64_t tile = pre ? segment_tile<P, true>() : segment_tile<P, false>();
  const auto prepare = [&] {
    if (!fill_kargs<P>(c, nbufs, a.k, true) || !segments_valid(segs, n_segs, c.T)) {
      return false;
    }
    a.k.g = Grid{c.T, 0, 0, 0, 0, 0, 0, 0};
    vec_rows = rows_streamable<P>(a.k.x, nbufs, a.k.g.res0, a.k.g.rmod);
    const int nth = pre ? segment_threads<P, true>() : segment_threads<P, false>();
    return walk_fits<T>(walk, c.R, tile, vec_rows, a.seg, nth);
  };
  return run_step<P>(c, a.k.vec, prepare, [&]() -> int {
    const bool same_phase =
        rows_same_phase<P>(a.k.x, nbufs, stream_pack<typename P::T, typename P::S>());
    if constexpr (P::kPreWords > 0) {
      if (pre) {
        constexpr int nth = segment_threads<P, true>();
        // the cap only where it can pay (as for the streaming driver's
        // launches: at least kCapMinElems elements)
        const uint32_t lds =
            c.R * c.T >= kCapMinElems ? segment_lds_pre_of<P>::value : 0u;
        return same_phase ? launch_walk<T>(walk, c.R, tile, vec_rows, a, a.seg,
                                           segment_kernel<P, false, true>, c.stream, lds, nth)
                          : launch_walk<T>(walk, c.R, tile, vec_rows, a, a.seg,
                                           segment_kernel<P, true, true>, c.stream, lds, nth);
      }
    }
    constexpr int nth = segment_threads<P, false>();
    return same_phase ? launch_walk<T>(walk, c.R, tile, vec_rows, a, a.seg,
                                       segment_kernel<P, false, false>, c.stream, 0, nth)
                      : launch_walk<T>(walk, c.R, tile, vec_rows, a, a.seg,
                                       segment_kernel<P, true, false>, c.stream, 0, nth);
  });
}

inline Call make_call(const ts_rt_buf* bufs, void* steps, std::initializer_list<const void*> h,
                      const uint8_t* mask, int64_t R, int64_t T, uint32_t flags,
                      void* out_zero, void* stream, void* ws = nullptr, size_t ws_bytes = 0) {
  Call c;
  c.ws = ws;
  c.ws_bytes = ws_bytes;
  c.bufs = bufs;
  c.steps = steps;
  c.nh = 0;
  for (const void* p : h) c.h[c.nh++] = p;
  c.mask = mask;
  c.R = R;
  c.T = T;
  c.flags = flags;
  c.out_zero = out_zero;
  c.stream = static_cast<hipStream_t>(stream);
  return c;
}

}  // namespace
}  // namespace churten
