// Launch order of the QKV projection's tiles (qkv_proj.hip), host and device.
// Plain C++ as well, so a CPU test can check that every XCD's list together
// covers every tile exactly once.
#pragma once

#ifndef __HIPCC__
#define __host__
#define __device__
#endif

namespace h3hip {

constexpr int kOrderChunk = 4;   // token tiles per chunk
constexpr int kOrderXcds = 8;    // MI355X: 8 XCDs, workgroups dispatched round-robin

// Launch order of the (token tile, channel tile) grid. A chunk is kOrderChunk
// token tiles of one channel tile; chunk c = g * tiles_n + tn covers token
// tiles kOrderChunk g .. (the last group may be short). Chunk c belongs to XCD
// c % 8, which runs its chunks in order of c. So at any time the 8 XCDs work
// on the same few token tiles, each on its own channel tiles: x is fetched
// from HBM about once and shared through the last-level cache, W stays
// resident there, and each XCD's 32 concurrent workgroups (8 chunks) share 4
// x slices and 8 W slices per step in its L2. An order in which each XCD
// sweeps all channel tiles of its own token rows keeps more of x and W in
// flight than the 256 MB last-level cache holds at hidden 5120.
struct TileOrder {
  int tiles_m, tiles_n;
  // Chunks c < n with c % 8 == x.
  __host__ __device__ int count(int n, int x) const { return n > x ? (n - 1 - x) / kOrderXcds + 1 : 0; }
  __host__ __device__ int full_chunks() const { return (tiles_m / kOrderChunk) * tiles_n; }
  __host__ __device__ int all_chunks() const { return ((tiles_m + kOrderChunk - 1) / kOrderChunk) * tiles_n; }
  // Tiles XCD x runs.
  __host__ __device__ int length(int x) const {
    const int nf = full_chunks();
    return kOrderChunk * count(nf, x) + (tiles_m % kOrderChunk) * (count(all_chunks(), x) - count(nf, x));
  }
  // The p-th tile (p < length(x)) XCD x runs, as token tile << 16 | channel tile.
  __host__ __device__ int tile(int x, int p) const {
    const int nf = full_chunks(), fx = count(nf, x);
    int c, i;
    if (p < kOrderChunk * fx) {
      c = x + kOrderXcds * (p / kOrderChunk);
      i = p % kOrderChunk;
    } else {   // the short chunks of the last group, tiles_m % kOrderChunk tiles each
      const int r = tiles_m % kOrderChunk, q = p - kOrderChunk * fx;
      c = nf + ((x - nf) % kOrderXcds + kOrderXcds) % kOrderXcds + kOrderXcds * (q / r);
      i = q % r;
    }
    return (kOrderChunk * (c / tiles_n) + i) << 16 | (c % tiles_n);
  }
};

}  // namespace h3hip
