// Cube-sphere halo fill and crop for gfx950 (bandwidth-bound gathers).
//
// pad: [L, 6, n, n] -> [L, 6, S, S], S = n + 2p.  Every output cell is one of
//   interior  -> the face's own cell;
//   halo      -> a cell of the neighbouring face: the host composes the
//                neighbour table, the edge strip and its two quarter turns
//                into one affine map per (face, side), (x, y) = c + A (u, v)
//                with (u, v) the cell's place in the side's halo block;
//   corner    -> from the halo column (one value per row) and the halo row
//                (one value per column) beside it, split by the corner's
//                diagonal, their mean on it.
// crop: [L, 6, S, S] -> [L, 6, S - 2h, S - 2h], the centre.
// Each thread writes one 16-byte run of an output row (grid y/z = plane), so
// stores are 16-byte and coalesced; interior loads coalesce too, rotated halo
// strips read down columns of the neighbour (L2-resident: the next row's
// threads read the neighbouring elements of the same lines).
#include "common.h"

namespace strata {

enum { SIDE_TOP = 0, SIDE_RIGHT = 1, SIDE_BOTTOM = 2, SIDE_LEFT = 3 };

struct HaloMap {
  int nbr;
  int c0, c1;            // source (x, y) of halo-block cell (0, 0)
  int a00, a01, a10, a11;  // d(x, y) / d(u, v)
};

struct CubeParams {
  const void* src;
  void* dst;
  int64_t L;
  int n, p, S;
  int vec;  // rows start 16-byte aligned: whole runs use one 16-byte store
  HaloMap map[6][4];
};

template <typename T>
__device__ __forceinline__ float to_f(T v) { return (float)v; }

template <typename T>
__device__ __forceinline__ T halo_value(const CubeParams& q, const T* src, int64_t l, int f, int i, int j) {
  const int n = q.n, p = q.p;
  int side, u, v;
  if (i >= p + n) { side = SIDE_TOP; u = i - p - n; v = j - p; }
  else if (i < p) { side = SIDE_BOTTOM; u = i; v = j - p; }
  else if (j < p) { side = SIDE_LEFT; u = i - p; v = j; }
  else { side = SIDE_RIGHT; u = i - p; v = j - p - n; }
  const HaloMap& m = q.map[f][side];
  const int x = m.c0 + m.a00 * u + m.a01 * v;
  const int y = m.c1 + m.a10 * u + m.a11 * v;
  return src[((l * 6 + m.nbr) * n + x) * (int64_t)n + y];
}

template <typename T>
__device__ __forceinline__ T mean2(T a, T b);
template <>
__device__ __forceinline__ float mean2<float>(float a, float b) { return (a + b) / 2.f; }
template <>
__device__ __forceinline__ bf16 mean2<bf16>(bf16 a, bf16 b) {
  const bf16 s = (bf16)((float)a + (float)b);  // bf16 + bf16 rounds to bf16, then an exact halving
  return (bf16)((float)s * 0.5f);
}

// Value of padded cell (i, j) of plane (l, f).
template <typename T>
__device__ __forceinline__ T pad_value(const CubeParams& q, const T* src, int64_t l, int f, int i, int j) {
  const int n = q.n, p = q.p;
  const bool bi = i >= p && i < p + n, bj = j >= p && j < p + n;
  if (bi && bj) return src[((l * 6 + f) * n + (i - p)) * (int64_t)n + (j - p)];
  if (bi || bj) return halo_value<T>(q, src, l, f, i, j);
  // corner: local (a, b) in [0, p)^2; v from the halo column beside it, h from the halo row
  const bool top = i >= p + n, right = j >= p + n;
  const int a = top ? i - p - n : i, b = right ? j - p - n : j;
  const int vc = right ? p + n - 1 : p, hr = top ? p + n - 1 : p;
  const T v = halo_value<T>(q, src, l, f, i, vc);
  const T h = halo_value<T>(q, src, l, f, hr, j);
  // bottom-left / top-right: main diagonal; the other two: anti-diagonal.  v
  // takes the side "above" (a < b, or a + b < p - 1) in the bottom corners and
  // the side "below" in the top corners.
  const bool main = top == right;
  const int sgn = main ? (a < b ? 1 : (a > b ? -1 : 0)) : (a + b < p - 1 ? 1 : (a + b > p - 1 ? -1 : 0));
  const int vsgn = top ? -1 : 1;
  return sgn == 0 ? mean2<T>(v, h) : (sgn == vsgn ? v : h);
}

// Pad, one launch per call; grid x = [interior runs | halo tiles | corner
// cells] of one plane, grid y/z = the L * 6 planes.
//  - interior: 16-byte runs of the face copied into the centre;
//  - halo: 32 x 32 tiles of each side's halo block; the tile's source is a
//    32 x 32 block of the neighbour face (the side's map is a signed
//    permutation), read row by row into LDS and written out row by row, so
//    both the reads and the writes coalesce whatever the quarter turn;
//  - corners: one cell per thread from the two halo lines beside it.
constexpr int CT = 32;  // halo tile side

struct PadLayout {
  int int_blocks;     // interior blocks (256 runs each)
  int halo_blocks[5]; // prefix sums of the tiles of the 4 sides
  int corner_blocks;
};

template <typename T>
__device__ __forceinline__ void halo_tile(const CubeParams& q, const T* src, T* dst, int64_t l, int f, int side,
                                          int tile, T (*sm)[CT + 1]) {
  const int n = q.n, p = q.p, S = q.S;
  const bool tb = side == SIDE_TOP || side == SIDE_BOTTOM;
  const int hu = tb ? p : n, hv = tb ? n : p;  // halo block shape
  const int ntv = (hv + CT - 1) / CT;
  const int u0 = (tile / ntv) * CT, v0 = (tile % ntv) * CT;
  const int tu = min(CT, hu - u0), tv = min(CT, hv - v0);
  const HaloMap& m = q.map[f][side];
  // source block: the image of [u0, u0 + tu) x [v0, v0 + tv)
  const int xa = m.c0 + m.a00 * u0 + m.a01 * v0, xb = m.c0 + m.a00 * (u0 + tu - 1) + m.a01 * (v0 + tv - 1);
  const int ya = m.c1 + m.a10 * u0 + m.a11 * v0, yb = m.c1 + m.a10 * (u0 + tu - 1) + m.a11 * (v0 + tv - 1);
  const int x0 = min(xa, xb), y0 = min(ya, yb), sx = max(xa, xb) - x0 + 1, sy = max(ya, yb) - y0 + 1;
  const T* sp = src + (l * 6 + m.nbr) * (int64_t)n * n;
  const int tx = threadIdx.x & (CT - 1), ty = threadIdx.x / CT;  // 32 x 8 threads
  for (int r = ty; r < sx; r += 256 / CT) {
    if (tx < sy) {
      const int x = x0 + r, y = y0 + tx;
      const int dx = x - m.c0, dy = y - m.c1;
      const int u = m.a00 * dx + m.a10 * dy, v = m.a01 * dx + m.a11 * dy;  // A^T: the map is orthogonal
      sm[u - u0][v - v0] = sp[(int64_t)x * n + y];
    }
  }
  __syncthreads();
  T* dp = dst + (l * 6 + f) * (int64_t)S * S;
  const int ro = side == SIDE_TOP ? p + n : side == SIDE_BOTTOM ? 0 : p;
  const int co = side == SIDE_LEFT ? 0 : side == SIDE_RIGHT ? p + n : p;
  for (int r = ty; r < tu; r += 256 / CT)
    if (tx < tv) dp[(int64_t)(ro + u0 + r) * S + co + v0 + tx] = sm[r][tx];
}

template <typename T>
__global__ __launch_bounds__(256) void cube_pad_kernel(CubeParams q, PadLayout lay) {
  constexpr int V = 16 / sizeof(T);
  __shared__ T sm[CT][CT + 1];
  const int64_t plane = blockIdx.y + (int64_t)gridDim.y * blockIdx.z;
  if (plane >= q.L * 6) return;  // uniform over the block
  const T* src = (const T*)q.src;
  T* dst = (T*)q.dst;
  const int64_t l = plane / 6;
  const int f = (int)(plane - l * 6);
  const int n = q.n, p = q.p, S = q.S;
  int b = blockIdx.x;
  if (b < lay.int_blocks) {
    const int runs = (n + V - 1) / V;
    const int t = b * 256 + threadIdx.x;
    if (t >= n * runs) return;
    const int i = t / runs, j0 = (t - i * runs) * V;
    const T* in = src + (plane * n + i) * (int64_t)n + j0;
    T* out = dst + (plane * S + p + i) * (int64_t)S + p + j0;
    if (q.vec && j0 + V <= n) {
      *(u32x4*)out = *(const u32x4*)in;
    } else {
      for (int e = 0; e < V && j0 + e < n; ++e) out[e] = in[e];
    }
    return;
  }
  b -= lay.int_blocks;
  if (b < lay.halo_blocks[4]) {
    int side = 0;
    while (b >= lay.halo_blocks[side + 1]) ++side;
    halo_tile<T>(q, src, dst, l, f, side, b - lay.halo_blocks[side], sm);
    return;
  }
  b -= lay.halo_blocks[4];
  const int c = b * 256 + threadIdx.x;  // corner cell: 4 corners of p x p
  if (c >= 4 * p * p) return;
  const int k = c / (p * p), a = (c / p) % p, bb = c % p;
  const bool top = k >= 2, right = k & 1;
  const int i = top ? p + n + a : a, j = right ? p + n + bb : bb;
  dst[(plane * S + i) * (int64_t)S + j] = pad_value<T>(q, src, l, f, i, j);
}

template <typename T>
__global__ __launch_bounds__(256) void cube_crop_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t planes,
                                                       int S, int h, int vec) {
  constexpr int V = 16 / sizeof(T);
  const int64_t plane = blockIdx.y + (int64_t)gridDim.y * blockIdx.z;
  if (plane >= planes) return;
  const int C = S - 2 * h, runs = (C + V - 1) / V;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= C * runs) return;
  const int i = t / runs, j0 = (t - i * runs) * V;
  const T* in = src + (plane * S + i + h) * (int64_t)S + h + j0;
  T* out = dst + (plane * C + i) * (int64_t)C + j0;
  if (vec && j0 + V <= C) {
    T vals[V];
#pragma unroll
    for (int e = 0; e < V; ++e) vals[e] = in[e];
    *(u32x4*)out = *(const u32x4*)vals;
  } else {
    for (int e = 0; e < V && j0 + e < C; ++e) out[e] = in[e];
  }
}

// Launch shape for `planes` planes of `rows` x `runs` 16-byte runs.
static dim3 plane_grid(int64_t planes, int64_t cells) {
  const int64_t y = planes < 65535 ? planes : 65535;
  return dim3((unsigned)((cells + 255) / 256), (unsigned)y, (unsigned)((planes + y - 1) / y));
}

// ---------------------------------------------------------------------------
// Host: the halo maps
// ---------------------------------------------------------------------------
// Neighbour table (screamcast/cubesphere_transforms.py:149-196):
// kNbr[face][side] = {neighbour face, neighbour edge}, sides/edges indexed
// top, right, bottom, left.
static const int kNbr[6][4][2] = {
    {{5, SIDE_BOTTOM}, {1, SIDE_LEFT}, {4, SIDE_TOP}, {3, SIDE_RIGHT}},
    {{5, SIDE_RIGHT}, {2, SIDE_LEFT}, {4, SIDE_RIGHT}, {0, SIDE_RIGHT}},
    {{5, SIDE_TOP}, {3, SIDE_LEFT}, {4, SIDE_BOTTOM}, {1, SIDE_RIGHT}},
    {{5, SIDE_LEFT}, {0, SIDE_LEFT}, {4, SIDE_LEFT}, {2, SIDE_RIGHT}},
    {{0, SIDE_BOTTOM}, {1, SIDE_BOTTOM}, {2, SIDE_BOTTOM}, {3, SIDE_BOTTOM}},
    {{2, SIDE_TOP}, {1, SIDE_TOP}, {0, SIDE_TOP}, {3, SIDE_TOP}},
};
// Quarter turns (torch.rot90 k over the last two dims): an edge strip to the
// canonical (p, n) strip (:229-252) and the canonical strip to a side (:255-273).
static int k_to_canonical(int edge) {
  return edge == SIDE_BOTTOM ? 0 : edge == SIDE_LEFT ? -1 : edge == SIDE_RIGHT ? 1 : 2;
}
static int k_to_side(int side) { return side == SIDE_TOP ? 0 : side == SIDE_RIGHT ? 1 : side == SIDE_LEFT ? -1 : 2; }

// Position in rot90(in, k) -> position in `in` (shape H x W).
static void rot_back(int k, int H, int W, int i, int j, int& ii, int& jj) {
  k = ((k % 4) + 4) % 4;
  if (k == 0) { ii = i; jj = j; }
  else if (k == 1) { ii = j; jj = W - 1 - i; }
  else if (k == 2) { ii = H - 1 - i; jj = W - 1 - j; }
  else { ii = H - 1 - j; jj = i; }
}

// Source cell of halo-block cell (u, v) of (face, side).
static void halo_source(int face, int side, int n, int p, int u, int v, int& x, int& y) {
  const int edge = kNbr[face][side][1];
  const bool tb = edge == SIDE_TOP || edge == SIDE_BOTTOM;
  const int RH = tb ? p : n, RW = tb ? n : p;  // raw strip shape
  int ci, cj, ri, rj;
  rot_back(k_to_side(side), p, n, u, v, ci, cj);              // canonical strip is p x n
  const int kc = k_to_canonical(edge);
  rot_back(kc, RH, RW, ci, cj, ri, rj);
  x = ri + (edge == SIDE_TOP ? n - p : 0);
  y = rj + (edge == SIDE_RIGHT ? n - p : 0);
}

static void build_maps(CubeParams& q) {
  for (int f = 0; f < 6; ++f)
    for (int s = 0; s < 4; ++s) {
      HaloMap& m = q.map[f][s];
      // the composition is affine: probe (0, 0), (1, 0), (0, 1) (outside a one-wide
      // block the formula still holds)
      int x0, y0, xu, yu, xv, yv;
      halo_source(f, s, q.n, q.p, 0, 0, x0, y0);
      halo_source(f, s, q.n, q.p, 1, 0, xu, yu);
      halo_source(f, s, q.n, q.p, 0, 1, xv, yv);
      m.nbr = kNbr[f][s][0];
      m.c0 = x0;
      m.c1 = y0;
      m.a00 = xu - x0;
      m.a10 = yu - y0;
      m.a01 = xv - x0;
      m.a11 = yv - y0;
    }
}

}  // namespace strata

using namespace strata;

extern "C" int strata_hip_cube_pad_faces(const strata_hip_cube_pad_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "cube_pad_faces: null args");
  if (a->dtype != STRATA_HIP_F32 && a->dtype != STRATA_HIP_BF16)
    return fail(STRATA_HIP_EINVAL, "cube_pad_faces: dtype must be f32 or bf16");
  if (a->lead < 0 || a->face_size <= 0 || a->pad < 0) return fail(STRATA_HIP_EINVAL, "cube_pad_faces: bad sizes");
  if (a->pad > a->face_size)
    return fail(STRATA_HIP_EINVAL, "cube_pad_faces: pad wider than a face (the halo is one neighbour's strip)");
  if (a->lead == 0) return STRATA_HIP_OK;
  if (!a->src || !a->dst) return fail(STRATA_HIP_EINVAL, "cube_pad_faces: null pointer");
  if (a->src == a->dst) return fail(STRATA_HIP_EINVAL, "cube_pad_faces: dst must not alias src");
  const int64_t S = (int64_t)a->face_size + 2 * a->pad;
  if ((int64_t)a->face_size * a->face_size > 0x7fffffff || S > 0x7fff)
    return fail(STRATA_HIP_EUNSUPPORTED, "cube_pad_faces: face too large");
  CubeParams q;
  q.src = a->src;
  q.dst = a->dst;
  q.L = a->lead;
  q.n = a->face_size;
  q.p = a->pad;
  q.S = (int)S;
  {  // interior runs: 16-byte loads and stores when every row of src and of dst's centre is aligned
    const int V = a->dtype == STRATA_HIP_F32 ? 4 : 8;
    q.vec = a->face_size % V == 0 && S % V == 0 && a->pad % V == 0 && ((uintptr_t)a->dst & 15) == 0 &&
            ((uintptr_t)a->src & 15) == 0;
  }
  build_maps(q);
  hipStream_t st = (hipStream_t)stream;
  const int V = a->dtype == STRATA_HIP_F32 ? 4 : 8;
  PadLayout lay;
  const int n = q.n, p = q.p;
  lay.int_blocks = (int)(((int64_t)n * ((n + V - 1) / V) + 255) / 256);
  const int tiles_tb = ((p + CT - 1) / CT) * ((n + CT - 1) / CT);  // top / bottom: p x n; left / right: n x p
  lay.halo_blocks[0] = 0;
  for (int s = 0; s < 4; ++s) lay.halo_blocks[s + 1] = lay.halo_blocks[s] + tiles_tb;
  lay.corner_blocks = (4 * p * p + 255) / 256;
  const int64_t blocks = (int64_t)lay.int_blocks + lay.halo_blocks[4] + lay.corner_blocks;
  const dim3 grid = plane_grid(a->lead * 6, blocks * 256);
  if (a->dtype == STRATA_HIP_F32)
    hipLaunchKernelGGL(cube_pad_kernel<float>, grid, dim3(256), 0, st, q, lay);
  else
    hipLaunchKernelGGL(cube_pad_kernel<bf16>, grid, dim3(256), 0, st, q, lay);
  return check_launch("cube_pad_kernel");
}

extern "C" int strata_hip_cube_crop(const strata_hip_cube_crop_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "cube_crop: null args");
  if (a->dtype != STRATA_HIP_F32 && a->dtype != STRATA_HIP_BF16)
    return fail(STRATA_HIP_EINVAL, "cube_crop: dtype must be f32 or bf16");
  if (a->planes < 0 || a->extent <= 0 || a->halo < 0 || 2 * (int64_t)a->halo >= a->extent)
    return fail(STRATA_HIP_EINVAL, "cube_crop: need planes >= 0 and 0 <= 2*halo < size");
  if (a->extent > 0x7fff) return fail(STRATA_HIP_EUNSUPPORTED, "cube_crop: extent too large");
  if (a->planes == 0) return STRATA_HIP_OK;
  if (!a->src || !a->dst) return fail(STRATA_HIP_EINVAL, "cube_crop: null pointer");
  const int64_t C = a->extent - 2 * (int64_t)a->halo;
  hipStream_t st = (hipStream_t)stream;
  const int V = a->dtype == STRATA_HIP_F32 ? 4 : 8;
  const dim3 grid = plane_grid(a->planes, C * ((C + V - 1) / V));
  const int vec = (C % V) == 0 && ((uintptr_t)a->dst & 15) == 0;
  if (a->dtype == STRATA_HIP_F32)
    hipLaunchKernelGGL(cube_crop_kernel<float>, grid, dim3(256), 0, st, (const float*)a->src, (float*)a->dst,
                       a->planes, a->extent, a->halo, vec);
  else
    hipLaunchKernelGGL(cube_crop_kernel<bf16>, grid, dim3(256), 0, st, (const bf16*)a->src, (bf16*)a->dst,
                       a->planes, a->extent, a->halo, vec);
  return check_launch("cube_crop_kernel");
}
