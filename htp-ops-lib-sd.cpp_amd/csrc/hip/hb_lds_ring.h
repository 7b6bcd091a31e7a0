// Device helpers of the direct-to-LDS operand ring shared by the tiled MFMA
// GEMMs (int8 and fp16): operands are pre-arranged in HBM as 1 KB tiles in
// MFMA lane order, and one global_load_lds_dwordx4 per wave fills one tile.
// Included inside each translation unit's anonymous namespace.
#ifndef HB_LDS_RING_H
#define HB_LDS_RING_H

constexpr int kRingTileBytes = 1024;  // one 16-row operand tile (16 x 64 int8 or 16 x 32 fp16)

#define HB_LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ inline void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Waits until at most `ahead` later stages (PW DMA instructions each) are
// still in flight for this wave; ahead <= A.
template <int PW, int A>
__device__ inline void wait_stage(int ahead) {
  if constexpr (A == 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= A) {
      wait_vmcnt<A * PW>();
    } else {
      wait_stage<PW, A - 1>(ahead);
    }
  }
}

// Tile p of the grid walked in groups of 4 row blocks, column by column.
__device__ inline void group_tile(int p, int tiles_m, int tiles_n, int &tm, int &tn) {
  constexpr int G = 4;
  const int first_m = (p / (G * tiles_n)) * G;
  const int gsize = min(tiles_m - first_m, G);
  const int in_group = p % (G * tiles_n);
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// Workgroups are dispatched round-robin over the 8 XCDs: tile ids are first
// made contiguous per XCD, then walked in groups of 4 row-blocks so that
// workgroups resident together on one XCD share A and B blocks in its L2.
__device__ inline void tile_coords(int bid, int tiles_m, int tiles_n, int &tm, int &tn) {
  const int total = tiles_m * tiles_n;
  const int pid = (total % 8 == 0) ? (bid % 8) * (total / 8) + bid / 8 : bid;
  group_tile(pid, tiles_m, tiles_n, tm, tn);
}

// Tile of workgroup bid for kernels of one tile per workgroup, XCD-aware in
// two dimensions: each of the 8 XCDs (bid % 8) owns one of pm x (8 / pm)
// equal rectangles of the tile grid, pm chosen to minimise the operand bytes
// a rectangle touches (rows * BM + columns * BN, both operands being of one
// element size), walked in groups of 4 row blocks column by column.  An
// XCD then reads only its rectangle's row and column blocks, where the
// 1-D chunks of tile_coords make every XCD read most of the wider operand.
// Falls back to tile_coords when no split divides the grid evenly.
template <int BM, int BN>
__device__ inline void tile_coords_2d(int bid, int tiles_m, int tiles_n, int &tm, int &tn) {
  int pm = 0, best = -1;
#pragma unroll
  for (int p = 1; p <= 8; p *= 2) {
    if (tiles_m % p != 0 || tiles_n % (8 / p) != 0) continue;
    const int cost = (tiles_m / p) * BM + (tiles_n / (8 / p)) * BN;
    if (best < 0 || cost < best) {
      best = cost;
      pm = p;
    }
  }
  if (pm == 0) {
    tile_coords(bid, tiles_m, tiles_n, tm, tn);
    return;
  }
  const int pn = 8 / pm, rows = tiles_m / pm, cols = tiles_n / pn;
  const int xcd = bid % 8, p = bid / 8;  // p < rows * cols: the grid is rows * cols * 8 tiles
  constexpr int G = 4;
  const int first = (p / (G * cols)) * G;
  const int gsize = min(rows - first, G);
  const int in_group = p % (G * cols);
  tm = (xcd / pn) * rows + first + in_group % gsize;
  tn = (xcd % pn) * cols + in_group / gsize;
}

// Issues one stage's DMA: instruction i of this wave fills block i*NW + wave
// of the NB blocks of a stage (waves below NB % NW issue one more than the
// others when the blocks do not split evenly).
template <int PW, int NW, int NB = PW * NW>
__device__ inline void dma_stage(int8_t *stage, const int8_t *const *src, const int *stride, int kt,
                                 int wave, int lane) {
  (void)lane;
#pragma unroll
  for (int i = 0; i < PW; ++i)
    if (NB % NW == 0 || i * NW + wave < NB)
      __builtin_amdgcn_global_load_lds(src[i] + (size_t)kt * stride[i],
                                       HB_LDS_PTR(stage + (i * NW + wave) * kRingTileBytes), 16, 0, 0);
}


#endif  // HB_LDS_RING_H
