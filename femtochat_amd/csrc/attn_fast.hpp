// Building blocks of the bf16 (fast mode) kernels on gfx950.
//
// Global memory is read through buffer resources: one descriptor per
// (batch, head) slice whose record count ends at the slice's last valid byte,
// so a tile row at or beyond T reads as zero with no branch, and offsets are
// 32-bit.
//
// LDS tiles hold rows of D bf16 values in natural layout (row = token, the
// head dimension contiguous) with no padding; the 16-byte units of a row are
// XOR-swizzled by the row index:  unit u of row r lives at unit u ^ swz(r),
// swz(r) = 4(r mod 4) + (r/4 mod 4)   (masked to the row's unit count).
// With D = 128 (16 units = one pass over the 64 banks per row) this makes
//   * a natural fragment read (16 lanes, 16 consecutive rows, one unit) and
//   * a transposed read with ds_read_b64_tr_b16 (32 lanes, 4 consecutive rows,
//     units 4k..4k+3)
// both free of bank conflicts, so one copy of a tile serves both operand
// orientations.
//
// ds_read_b64_tr_b16 (gfx950): within each block of 16 lanes, lane s supplies
// the address of 4 consecutive 16-bit values; output lane i receives value
// (i mod 4) of the chunks of lanes i/4, 4 + i/4, 8 + i/4, 12 + i/4.  Lane s =
// 4a + c pointing at X[k0 + a][n0 + 4c] therefore hands lane i the column
// n0 + i, rows k0..k0+3: a 4 x 16 transpose per instruction.
#pragma once

#include "attn_device.hpp"

namespace fc {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr uint32_t kBufferWord3 = 0x00020000u;  // raw buffer, 32-bit data format

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kBufferWord3);
}

// Descriptor for the rows from byte row0 of a slice of `records` valid bytes.
// The range check covers the per-lane offset only (not the scalar offset), so
// a tile gets its own descriptor rather than a scalar offset.
__device__ inline __amdgpu_buffer_rsrc_t tile_rsrc(const char* base, int64_t records, int64_t row0) {
  const int64_t left = records - row0;
  return make_rsrc(base + row0, (uint32_t)(left > 0 ? left : 0));
}

__device__ inline uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

template <int D>
struct SwzTile {
  static constexpr int kUPR = D / 8;          // 16-byte units per row
  static constexpr int kRowBytes = 2 * D;
  __device__ static constexpr int swz(int r) { return (4 * (r & 3) + ((r >> 2) & 3)) & (kUPR - 1); }
  __device__ static constexpr int offset(int r, int u) { return r * kRowBytes + 16 * (u ^ swz(r)); }
};

// Which key bounds a masked tile body tests: kLower (key >= the row's lower
// bound), kUpper (key <= its upper bound) or both; a tile that no row's
// upper bound cuts (all its keys at or below every row's ub) needs no upper
// test, and likewise for the lower bound.
constexpr int kLower = 1, kUpper = 2, kBoth = kLower | kUpper;

// 16 bytes at a byte offset of an LDS buffer.
__device__ inline uint4 lds_load16(const char* lds, int off) { return *reinterpret_cast<const uint4*>(lds + off); }
__device__ inline void lds_store16(char* lds, int off, uint4 v) { *reinterpret_cast<uint4*>(lds + off) = v; }

__device__ inline bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// Fragment (accumulator k order) from two transposed 8-byte reads.
__device__ inline bf16x8 lds_tr_frag(const char* lds, int off0, int off1) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds + off0));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds + off1));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  s16x8 v;
  v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
  v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
  return __builtin_bit_cast(bf16x8, v);
}

// Per-lane byte offsets of fragment reads from a swizzled tile.
//   nat(c)    : natural fragment, row l32 (+32*k rows, added by the caller as
//               an immediate), 16-byte unit 2c+g.
//   tr(e, db) : transposed fragment, instruction e (rows 8e + 4(beta/2) + a,
//               + 16*kc rows by the caller), column block db (columns
//               32db + 16(beta%2) + 4c), beta = lane/16, a = (lane%16)/4,
//               c = lane%4.
// The swizzle only flips the bits that hold the unit index, so the offset of
// chunk c (or column block db) is one base XOR a constant: three registers
// per lane instead of a table.
template <int D>
struct FragOffsets {
  using Tile = SwzTile<D>;
  static constexpr int kKC = D / 16;
  static constexpr int kDB = D < 32 ? 1 : D / 32;
  int nat_base;
  int tr_base[2];

  __device__ inline void init(int lane) {
    const int g = lane >> 5, l32 = lane & 31;
    nat_base = Tile::offset(l32, g);  // chunk 0; chunk c is nat_base ^ 32c
    const int beta = lane >> 4, s = lane & 15, a = s >> 2, cc = s & 3;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = 8 * e + 4 * (beta >> 1) + a;  // row within a 16-row chunk
      int u = 2 * (beta & 1) + (cc >> 1);
      if (u > Tile::kUPR - 1) u = Tile::kUPR - 1;  // D < 32: lanes past D read a valid unit
      tr_base[e] = Tile::offset(r, u) + 8 * (cc & 1);  // column block 0; block db is ^ 64db
    }
  }
  __device__ inline int nat(int c) const { return nat_base ^ (32 * c); }
  __device__ inline int tr(int e, int db) const { return tr_base[e] ^ (64 * db); }
};

// Stages a tile of R rows x D bf16 (16-byte units) from global memory into a
// swizzled LDS tile.  StagePlan holds each thread's unit offsets (global,
// relative to the tile's first row, and LDS), shared by every tile of the
// same shape; StageRegs holds one tile's data in flight.
template <int D, int R, int NT>
struct StagePlan {
  using Tile = SwzTile<D>;
  static constexpr int kUnits = R * Tile::kUPR;
  static constexpr int kPer = (kUnits + NT - 1) / NT;
  int goff[kPer];
  int loff[kPer];

  __device__ inline void init(int tid, int pitch_bytes) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      int unit = tid + i * NT;
      if (unit >= kUnits) unit = kUnits - 1;  // duplicates a valid unit (same data, same slot)
      const int row = unit / Tile::kUPR, u = unit % Tile::kUPR;
      goff[i] = row * pitch_bytes + 16 * u;
      loff[i] = Tile::offset(row, u);
    }
  }
};

template <int D, int R, int NT>
struct StageRegs {
  using Plan = StagePlan<D, R, NT>;
  uint4 v[Plan::kPer];
  __device__ inline void load(const Plan& pl, __amdgpu_buffer_rsrc_t r) {
#pragma unroll
    for (int i = 0; i < Plan::kPer; ++i) v[i] = buf_load16(r, pl.goff[i], 0);
  }
  __device__ inline void store(const Plan& pl, char* lds) const {
#pragma unroll
    for (int i = 0; i < Plan::kPer; ++i) lds_store16(lds, pl.loff[i], v[i]);
  }
};

// Direct global -> LDS staging (buffer_load_dwordx4 ... lds, gfx950): one
// wave instruction writes 64 lanes x 16 bytes to a contiguous 1 KB block of
// LDS (lane l at M0 + 16 l) from per-lane global offsets, so the swizzle is
// applied on the global side: lane l of block i fills physical unit 64i + l,
// i.e. row (64i + l) / kUPR, logical unit (physical unit) ^ swz(row).  The
// data never passes through VGPRs.
//
// The load is issued from inline assembly so that the compiler does not treat
// every later LDS read as a possible alias of the transfer (it would wait for
// the transfer before the first one).  Completion is therefore the caller's
// job: dma_wait_barrier() waits for all of this wave's loads (vmcnt = 0) and
// then for the workgroup, before any wave reads the staged buffer.
typedef unsigned int u32x4s __attribute__((ext_vector_type(4)));

// Raw buffer descriptor words: base (48 bits), stride 0, record count, flags.
__device__ inline u32x4s buffer_words(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  u32x4s w;
  w[0] = (uint32_t)p;
  w[1] = (uint32_t)(p >> 32) & 0xffffu;
  w[2] = bytes;
  w[3] = kBufferWord3;
  return w;
}

__device__ inline u32x4s tile_words(const char* base, int64_t records, int64_t row0) {
  const int64_t left = records - row0;
  return buffer_words(base + row0, (uint32_t)(left > 0 ? left : 0));
}

__device__ inline void dma_load16(u32x4s words, int voff, uint32_t lds_addr) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(words), "{m0}"(lds_addr) : "memory");
}

// The same for 4 bytes per lane (a 256-byte block of LDS).
__device__ inline void dma_load4(u32x4s words, int voff, uint32_t lds_addr) {
  asm volatile("buffer_load_dword %0, %1, 0 offen lds" : : "v"(voff), "s"(words), "{m0}"(lds_addr) : "memory");
}

// Waits until at most n of this wave's global loads (LDS-DMA included) are
// outstanding; loads complete in issue order, so the older ones have landed.
__device__ inline void wait_vmcnt(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
  }
}

template <int D, int R, int NW = kWaves>
struct DmaPlan {
  using Tile = SwzTile<D>;
  static constexpr int kInstr = R * Tile::kUPR / 64;  // 1 KB blocks per tile
  static_assert(R * Tile::kUPR % 64 == 0, "tile must be a whole number of 1 KB blocks");
  static constexpr int kPerWave = (kInstr + NW - 1) / NW;
  int goff[kPerWave];

  __device__ inline void init(int wave, int lane, int pitch_bytes) {
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
      const int i = wave + NW * j;
      const int P = 64 * i + lane;
      const int row = P / Tile::kUPR, pu = P % Tile::kUPR;
      goff[j] = row * pitch_bytes + 16 * (pu ^ Tile::swz(row));
    }
  }
  // Issues this wave's share of one tile's loads into the LDS tile at lds_addr.
  __device__ inline void issue(u32x4s words, uint32_t lds_addr, int wave) const {
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) issue_one(words, lds_addr, wave, j);
  }
  // The j-th of them, for callers that spread the loads over their compute;
  // j >= kPerWave issues nothing.
  __device__ inline void issue_one(u32x4s words, uint32_t lds_addr, int wave, int j) const {
    const int i = wave + NW * j;
    if (j < kPerWave && (kInstr % NW == 0 || i < kInstr))
      dma_load16(words, goff[j], __builtin_amdgcn_readfirstlane(lds_addr + 1024 * i));
  }
  // Number of loads issue() makes on wave `wave`.
  __host__ __device__ static constexpr int count(int wave) {
    int n = 0;
    for (int j = 0; j < kPerWave; ++j) n += (wave + NW * j < kInstr) ? 1 : 0;
    return n;
  }
};

// LDS byte address of a __shared__ object (the value M0 expects).
__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Waits for this wave's outstanding global loads (including LDS-DMA), then
// for every wave of the workgroup.
__device__ inline void dma_wait_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Orders the LDS accesses of one wave's lanes that exchange data through LDS
// (an epilogue's tile, written by every lane, read back by others): the
// writes before it are visible to the reads after it, and the reads before
// it complete before the writes after it.  The hardware runs one wave's LDS
// instructions in order, so no instruction is needed; without the fences the
// compiler treats each lane's accesses as its own and may move a read past
// other lanes' writes, or reuse an earlier read of the same address.
__device__ __attribute__((always_inline)) inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace fc
