// Workgroup -> (tile, head) mapping and host-side argument checks shared by
// the attention launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <initializer_list>
#include <string>

#include "tt_internal.h"

namespace tt {

// MI355X dispatches consecutive workgroup ids round-robin over its 8 XCDs,
// each with a private L2.  When the head count is a multiple of 8 the tiles
// of head bh all run on XCD bh % 8, and each XCD works through its heads in
// two phases:
//   1. heavy ranks (0 .. ntile - light - 1): `group` heads at a time, so the
//      K/V (or Q/dO) of the heads in flight stay in that L2; inside a group
//      the tile rank runs from the most expensive causal tile to cheaper ones;
//   2. the `light` cheapest ranks of every head of the XCD, heaviest first.
// Holding the short tiles of every head back to the end lets the XCD's
// workgroup slots finish together instead of waiting on the heavy tiles of
// the last head group (short tiles read little, so the lost L2 grouping
// costs little there).  `order` packs group | light << 16 (tile_order).
__host__ __device__ __forceinline__ void map_tile(int id, int ntile, int BH, int order, int& tile, int& bh,
                                         bool heavy_last) {
  const int group = order & 0xffff, light = order >> 16;
  int rank;
  if ((BH & 7) == 0 && group > 0) {
    const int xcd = id & 7, t = id >> 3, hx = BH >> 3;
    const int nh = ntile - light, heavy = hx * nh;
    if (t < heavy) {
      const int per = group * nh;
      const int gi = t / per, r = t - gi * per;
      rank = r / group;
      bh = xcd + 8 * (gi * group + (r - rank * group));
    } else {
      const int u = t - heavy;
      rank = nh + u / hx;
      bh = xcd + 8 * (u - (rank - nh) * hx);
    }
  } else {
    rank = id / BH;
    bh = id - rank * BH;
  }
  tile = heavy_last ? (ntile - 1 - rank) : rank;
}

// Largest divisor of BH/8 that keeps about `target` workgroups of one XCD on
// `group` heads at once (0 disables the XCD mapping).
inline int pick_group(int64_t BH, int64_t ntile, int64_t target) {
  if (BH % 8 != 0) return 0;
  int64_t per_xcd = BH / 8;
  int64_t want = target / (ntile > 0 ? ntile : 1);
  if (want < 1) want = 1;
  int64_t best = 1;
  for (int64_t gsz = 1; gsz <= per_xcd; ++gsz)
    if (per_xcd % gsz == 0 && gsz <= want) best = gsz;
  return (int)best;
}

// map_tile's `order` argument: the head group of pick_group and the
// ntile / light_div cheapest ranks held back to a final phase (light_div = 0:
// none; causal launches only, whose tiles differ in cost).  Measured on the
// MI355X with light_div = 2: the causal d = 64 kernels 3-6 % faster at
// L = 2048-8192, the [16,16,1024,64] step within +-3 % (its dK/dV kernel
// 2 % faster, the forward and dQ 1 % slower); at d = 128 the
// forward was 2 % slower (its light phase keeps the K/V of every head of the
// XCD in flight, several times the L2) and the [4,32,4096,128] step no faster
// (dQ -1.5 %, the dK/dV kernel after it slower), so d = 128 keeps the plain
// grouped order (attention_light_div).
inline int tile_order(int64_t BH, int64_t ntile, int64_t target, int light_div) {
  const int group = pick_group(BH, ntile, target);
  int64_t light = (light_div > 0 && group > 0) ? ntile / light_div : 0;
  if (light > 0x7fff) light = 0x7fff;  // any count <= ntile is a valid order
  return group | (int)(light << 16);
}

// light_div of the attention launches at head size d.
constexpr int attention_light_div(bool causal, int d) { return causal && d <= 64 ? 2 : 0; }

inline int check_attn_shape(const char* fn, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d,
                            int causal) {
  std::string f(fn);
  if (B < 0 || H < 0 || Lq < 0 || Lk < 0) return fail(TT_ERR_ARG, f + ": negative dimension");
  if (d != 32 && d != 64 && d != 128)
    return fail(TT_ERR_UNSUPPORTED, f + ": head dim must be 32, 64 or 128 (got " + std::to_string(d) + ")");
  if (causal && Lq != Lk) return fail(TT_ERR_ARG, f + ": causal mask needs Lq == Lk");
  if (Lq > 0 && Lk == 0 && B * H > 0) return fail(TT_ERR_ARG, f + ": softmax over zero keys");
  if (Lq > (int64_t(1) << 30) || Lk > (int64_t(1) << 30)) return fail(TT_ERR_ARG, f + ": sequence too long");
  if (B * H > (int64_t(1) << 24)) return fail(TT_ERR_ARG, f + ": too many heads");
  return TT_OK;
}

// Byte range of one launcher argument, for the overlap check below.
struct ArgSpan {
  const void* p;
  size_t bytes;
  const char* name;
};
inline bool spans_overlap(const ArgSpan& a, const ArgSpan& b) {
  if (!a.p || !b.p || a.bytes == 0 || b.bytes == 0) return false;
  const uintptr_t a0 = (uintptr_t)a.p, b0 = (uintptr_t)b.p;
  return a0 < b0 + b.bytes && b0 < a0 + a.bytes;
}
// Outputs may not overlap an input or another output: the kernels read their
// inputs while they write their outputs.  Inputs may overlap each other
// (q == k == v is a valid self-attention call).
inline int check_no_overlap(const char* fn, std::initializer_list<ArgSpan> inputs,
                            std::initializer_list<ArgSpan> outputs) {
  for (auto o = outputs.begin(); o != outputs.end(); ++o) {
    for (const ArgSpan& i : inputs)
      if (spans_overlap(*o, i))
        return fail(TT_ERR_ARG, std::string(fn) + ": output " + o->name + " overlaps input " + i.name);
    for (auto o2 = outputs.begin(); o2 != o; ++o2)
      if (spans_overlap(*o, *o2))
        return fail(TT_ERR_ARG, std::string(fn) + ": outputs " + o2->name + " and " + o->name + " overlap");
  }
  return TT_OK;
}

}  // namespace tt
