// fp32 GEMM and implicit-GEMM conv2d on gfx950 MFMA.
//
// Replaces the ijk double loop of __tensor_matmul__
// (modules/tensor/operators.cpp:757-766) and defines conv2d / dense on the
// same core.
//
// Main kernel (sgemm_kernel: one template, operand loaders for dense A/B,
// im2col gathers from NCHW, NHWC / NCHW4 k-quads and NCHW channel planes,
// v_mfma_f32_32x32x2_f32):
//   * work-group tile BM x BN, K consumed in stages of BK; WM x WN waves, each
//     owning (BM/WM) x (BN/WN) = FM x FN blocks of 32x32, optionally times WK
//     k-groups that split each stage's K and meet in LDS at the end;
//   * LDS holds both operands "k-quad major": plane q holds, for every row of
//     the tile, the 4 consecutive k values 4q..4q+3 as one 16-byte chunk, so a
//     lane fetches its 4 k values of a 32x32 block with one ds_read_b128;
//     planes are padded by 16 bytes, and B columns are XOR-swizzled (b_slot),
//     so that the stores and the operand reads are free of bank conflicts;
//   * a 32x32x2 MFMA takes, per lane l, k = 8s + 4*(l/32) + t (t = 0..3) from
//     that chunk: the lower half-wave covers k 0..3 of an 8-group, the upper
//     half k 4..7, and A and B use the same mapping, so every k is summed once;
//   * stages are double-buffered in LDS with the next stage held in registers
//     while the current one is multiplied, one barrier per stage;
//   * blockIdx is remapped so each of the 8 XCDs (own L2) works on a compact
//     group of tiles, grouped GROUP_M tile-rows deep (with K splits: on
//     whole splits);
//   * split-K (blockIdx.y) writes fp32 partials that tile_reduce_kernel sums in
//     split order and passes through the epilogue;
//   * epilogue: bias (per column for dense, per row = output channel for
//     conv) then relu as x * (x > 0), stored straight from the accumulators.
// Shapes the main kernel serves badly have their own kernels: N <= 32
// (sgemm_thin_kernel, fp32 FMA) and M <= 32 (sgemm_skinny_kernel, a
// streaming pass over B on v_mfma_f32_16x16x4_f32); conv2d with
// C*KH*KW <= 32 runs conv2d_direct_kernel.
#include "common.h"
#include "row_softmax.h"

#include <algorithm>
#include <type_traits>
#include <vector>

namespace camel_hip {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GROUP_M = 4;

// Operand loader kinds.  LOAD_CONV gathers im2col columns from NCHW x one
// float at a time; LOAD_NHWC reads x in NHWC with K ordered (kh, kw, c), so
// each k-quad of a pixel is one 16-byte load (needs C % BK == 0).
// LOAD_NHWC_POOL is LOAD_NHWC with the columns in pool-window order and a
// 2x2 max-pool epilogue (the fused conv2d..maxpool2d).  LOAD_PLANES and
// LOAD_PLANES_POOL read NCHW x in place with the same K order: a k-quad of a
// pixel is 4 loads from 4 channel planes, and a wave's lanes take consecutive
// pixels, so each load instruction reads a contiguous run of one plane.
// LOAD_TVEC / LOAD_TSCALAR (A operand only) read A given transposed, as
// At [K, M] row-major (A[m][k] = At[k][m]): like B, k rows with the tile's
// m contiguous, transposed 4x4 in registers before the LDS store, so
// transpose(X) @ E needs no copy of X (16-byte loads need M % 4 == 0).
// LOAD_DMA (A and B together, row-major, BK = 64 tiles whose stages are all
// inside M x N): each stage goes from global memory straight into LDS
// (global_load_lds_dwordx4, no registers and no LDS store instructions), A
// as rows of 64 k with k-quad q of tile row r in 16-byte slot (q + r) & 15
// (a 16-lane read of 16 rows' quad q touches 16 distinct bank groups), B as
// blocks of 4 k rows x BN columns stored as 64-column pieces, the 16-byte
// column chunks of odd blocks rotated by 8 (the half-waves read blocks q and
// q + 1: opposite halves of the 64 banks); the operand reads and the MFMA
// sequence are those of LOAD_VEC, so the results are bit-identical.
enum {
    LOAD_VEC = 0, LOAD_SCALAR = 1, LOAD_CONV = 2, LOAD_NHWC = 3, LOAD_NHWC_POOL = 4,
    LOAD_PLANES = 5, LOAD_PLANES_POOL = 6, LOAD_TVEC = 7, LOAD_TSCALAR = 8, LOAD_DMA = 9
};
template <int M> constexpr bool is_trans = (M == LOAD_TVEC || M == LOAD_TSCALAR);

// Loaders that take (pixel, k-quad) items over K ordered (kh, kw, c).
template <int M>
constexpr bool is_nhwc = (M == LOAD_NHWC || M == LOAD_NHWC_POOL || M == LOAD_PLANES ||
                          M == LOAD_PLANES_POOL);
template <int M> constexpr bool is_planes = (M == LOAD_PLANES || M == LOAD_PLANES_POOL);
template <int M> constexpr bool is_pool = (M == LOAD_NHWC_POOL || M == LOAD_PLANES_POOL);
template <int M> constexpr bool is_conv = (M == LOAD_CONV || is_nhwc<M>);

// Operands one call of a kernel's stage loader fetches.
enum LoadPart { LOAD_BOTH = 0, LOAD_A_ONLY = 1, LOAD_B_ONLY = 2 };
constexpr std::integral_constant<int, LOAD_BOTH> load_ab{};
constexpr std::integral_constant<int, LOAD_A_ONLY> load_a{};
constexpr std::integral_constant<int, LOAD_B_ONLY> load_b{};

// WK > 1 splits each stage's K range over WK groups of WM x WN waves (more
// waves per CU to hide latency when there are few tiles); the groups' sums
// meet in LDS at the end, added in group order.  EARLY selects the stage
// schedule with the barrier before the last 8-k group (see the main loop).
template <int BM_, int BN_, int BK_, int WM_, int WN_, int WK_ = 1, bool EARLY_ = true>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, WK = WK_;
    static constexpr bool EARLY = EARLY_;
    static constexpr int THREADS = 64 * WM * WN * WK;
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int FM = WTM / 32, FN = WTN / 32;
    static constexpr int KQ = BK / 4;
    static constexpr int A_PLANE = BM * 4 + 4;
    static constexpr int B_PLANE = BN * 4 + 4;
    static constexpr int A_STAGE = KQ * A_PLANE;
    static constexpr int B_STAGE = KQ * B_PLANE;
    static constexpr int STAGE = A_STAGE + B_STAGE;
    // LOAD_DMA stage: A as BM rows of BK floats, B as KQ blocks of 4 k rows
    // x BN floats, each block BN / 64 DMA pieces of 4 rows x 64 floats,
    // unpadded.
    static constexpr int DA_STAGE = BM * BK;
    static constexpr int DB_BLOCK = 4 * BN;
    static constexpr int D_STAGE = DA_STAGE + KQ * DB_BLOCK;
    // 16-byte load items per stage; a thread takes items tid + i * THREADS.
    static constexpr int A_TOTAL = BM * KQ;
    static constexpr int B_TOTAL = KQ * (BN / 4);
    static constexpr int BN_TOTAL = BN * KQ; // B as pixel rows (LOAD_NHWC)
    static constexpr int A_T_TOTAL = KQ * (BM / 4); // A given transposed: 4 k rows x 4 m
    static constexpr int A_ITEMS = (A_TOTAL + THREADS - 1) / THREADS;
    static constexpr int A_T_ITEMS = (A_T_TOTAL + THREADS - 1) / THREADS;
    static constexpr int B_ITEMS = (B_TOTAL + THREADS - 1) / THREADS;
    static constexpr int BN_ITEMS = (BN_TOTAL + THREADS - 1) / THREADS;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
    static_assert(BN % 32 == 0, "B column swizzle works on aligned runs of 32 columns");
    static_assert(BK % (8 * WK) == 0, "each wave k-group takes whole 8-k groups of a stage");
    static_assert(A_TOTAL % 64 == 0 && B_TOTAL % 64 == 0, "item guards must be wave-uniform");
    static_assert(A_T_TOTAL % 64 == 0, "transposed-A item guards must be wave-uniform");
    static_assert((WK - 1) * BM * BN <= 2 * STAGE, "k-group reduction must fit the LDS buffers");
};

struct GemmArgs {
    const float *A;  // [M, lda] row-major (conv: weights [Co, C*KH*KW]); transposed
                     // loaders: At [K, lda] row-major with lda >= M
    const float *B;  // [K, ldb] row-major (conv: input x, NCHW)
    float *C;        // [M, ldc] row-major (conv: output y, NCHW)
    const float *bias;
    float *partial;  // split-K partials [split][tile of launch][BM * BN], or null
    const int2 *ktab; // conv: per k {offset of (c,kh,kw) in x, kh << 16 | kw}
    int M, N, K;
    int lda, ldb, ldc;
    int k_per_split;  // multiple of BK
    int tile_begin;   // first logical tile of the launch
    int n_begin;      // first column of the launch's tile grid (a column band)
    int flags;
    // conv geometry (N = batch * P columns); Cin, KW, pxs, cqs only for
    // LOAD_NHWC.  The channel-quad input layouts it reads put channels
    // 4q .. 4q+3 of pixel (ih, iw) of image n at the 16 bytes starting at
    // n * CHW + (ih * W + iw) * pxs + q * cqs floats: NHWC has pxs = Cin,
    // cqs = 4; NCHW4 ([N][C/4][H][W][4]) has pxs = 4, cqs = 4 * H * W.
    int P, OW, H, W, CHW, stride, pad;
    int Cin, KW, pxs, cqs;
    // LOAD_NHWC_POOL: columns in pool order, 4 per window of a 2x2 stride-2
    // max pool over a PH x PW grid (PP = PH * PW windows per image); C is the
    // pooled output [batch][M][PP]
    int PW, PP;
    // LOAD_PLANES: distance between channel planes (H * W); pxs = 1 and
    // cqs = 4 * H * W
    int chs;
    // Classifier head (64 x 64 tiles, row-major operands): instead of C, each
    // tile stores its columns' share of the next layer's products,
    // head_partial[tn][m][n] = sum_j C[m][64 tn + j] * head_w[64 tn + j][n]
    // (j ascending) for n < head_n2 <= 16, where C is the finished tile (bias,
    // relu); null for an ordinary GEMM.
    const float *head_w;
    float *head_partial;
    int head_n2;
};

// Tiles whose epilogue can run the classifier head (GemmArgs::head_w).
template <class T, int AMODE, int BMODE>
constexpr bool head_tile = T::BM == 64 && T::BN == 64 && T::WK == 2 && T::FM == 1 && T::FN == 1 &&
                           ((AMODE == LOAD_VEC && BMODE == LOAD_VEC) ||
                            (AMODE == LOAD_DMA && BMODE == LOAD_DMA));
constexpr int HEAD_MAX_N2 = 16;

// (pixel, k-quad) of B item q of a stage: NHWC-style loaders put a pixel's
// k-quads on consecutive lanes (one 16-byte load each); the plane loaders put
// consecutive pixels on consecutive lanes.
template <class T, int BMODE> __device__ __forceinline__ int item_pixel(int q) {
    return is_planes<BMODE> ? q % T::BN : q / T::KQ;
}
template <class T, int BMODE> __device__ __forceinline__ int item_kquad(int q) {
    return is_planes<BMODE> ? q / T::BN : q % T::KQ;
}

// Value of lane Q of this lane's quad (lanes 4i .. 4i+3): a DPP quad_perm
// move, one VALU op with no LDS traffic.
template <int Q> __device__ __forceinline__ float quad_lane(float v) {
    constexpr int ctrl = Q | (Q << 2) | (Q << 4) | (Q << 6);
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xf, 0xf, false));
}

// Offset of conv output (image img, channel row, pixel p) in y: NCHW, or
// NCHW4 ([N][M/4][P][4], M % 4 == 0) for q4.
__device__ __forceinline__ size_t conv_out_off(const GemmArgs &g, bool q4, int img, int row, int p) {
    return q4 ? (size_t)img * g.M * g.P + (size_t)(row & ~3) * g.P + 4 * (size_t)p + (row & 3)
              : ((size_t)img * g.M + row) * g.P + p;
}

// LDS slot of B column n within a k-quad plane.  A 16-byte LDS access is
// served 8 lanes at a time over the 32 banks; the register-transposed B
// stores have lanes 4 columns apart (n = 4 nq + c), which would put 8 lanes
// on 2 bank groups.  XOR-ing bits 0-1 with bits 3-4 spreads them over all 8,
// and keeps each aligned run of 8 columns (one 8-lane operand read) whole.
__device__ __forceinline__ int b_slot(int n) { return n ^ ((n >> 3) & 3); }

// Address of row k of a row-major operand with leading dimension ld, computed
// as an integer: k is below 0 for a ragged first stage, whose rows are never
// read (the loaders' guards), and no pointer outside the operand is formed by
// pointer arithmetic.
__device__ __forceinline__ const float *row_address(const float *base, int k, int ld) {
    return reinterpret_cast<const float *>(reinterpret_cast<uintptr_t>(base) +
                                           (size_t)k * ld * sizeof(float));
}

// Logical tile id -> (tm, tn), grouped GROUP_M tile-rows deep so that
// consecutive ids share B panels.  A bijection on [0, tiles_m * tiles_n).
__device__ __forceinline__ void tile_of(int id, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int per_group = GROUP_M * tiles_n;
    const int g = id / per_group;
    const int first_m = g * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    const int in_group = id - g * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// Inverse of tile_of: the logical tile id of tile (tm, tn).
__device__ __forceinline__ int tile_id(int tm, int tn, int tiles_m, int tiles_n) {
    const int g = tm / GROUP_M, first_m = g * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    return g * GROUP_M * tiles_n + tn * gsize + (tm - first_m);
}

// Position of this work-group: its tile (local to the launch, which covers
// tiles [tile_begin, tile_begin + gridDim.x)) and its K split (gridDim.y
// splits).  Work-groups are dispatched round-robin over the 8 XCDs in linear
// order (blockIdx.x fastest).  When the grid size nb is a multiple of 8, XCD x
// is given the contiguous range [x*nb/8, (x+1)*nb/8) of (split, tile)
// positions instead, so its L2 holds a compact block of tiles and, with K
// splits, whole splits: the A and B panels of one K range are fetched from
// HBM by one XCD rather than by every XCD that runs one of their tiles.
__device__ __forceinline__ void block_pos(int &local, int &split) {
    const int nt = gridDim.x, nb = nt * gridDim.y;
    int bid = blockIdx.x + nt * blockIdx.y;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    split = bid / nt;
    local = bid - split * nt;
}

// Tiles the LOAD_DMA stage loop serves (it has its own stage schedule):
// rows of 16 k-quads (one 16-lane row of a DMA instruction), B blocks of
// whole 64-column pieces, whole DMA instructions per wave.  Measured on the
// 64 x 64 tile (MLP, 1024^3, CNN dense1) and the one-round 128 x 128 tile
// with k-groups (2048^3).
template <class T>
constexpr bool dma_tile = T::BK == 64 && T::BN % 64 == 0 && T::BM % 64 == 0 && T::WK == 2 &&
                          (T::BM / 4) % (T::THREADS / 64) == 0 &&
                          (T::KQ * T::BN / 64) % (T::THREADS / 64) == 0;

// One 16-byte-per-lane LDS DMA (global_load_lds_dwordx4): lane l's 16
// bytes at src land at LDS address dst + 16 l, dst (in M0) wave-uniform.
// Inline assembly rather than the builtin: the compiler makes every LDS
// read after the builtin wait for it (vmcnt(0)), which would expose the
// whole DMA latency at the next operand read; here the loop's own
// vmcnt(0) before the stage barrier is the only wait (so nothing may read
// a stage's LDS before that barrier).  s_nop: the wait state an M0 write
// needs before an LDS DMA.
__device__ __forceinline__ uint32_t lds_address(const float *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float *)p;
}
__device__ __forceinline__ void dma16(const float *src, const float *dst) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds_address(dst)))
                 : "memory");
}
// Waits for this wave's outstanding vector memory loads, LDS DMAs included.
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <class T, int AMODE, int BMODE>
__global__ __launch_bounds__(T::THREADS) void sgemm_kernel(GemmArgs g) {
    constexpr bool DMA = AMODE == LOAD_DMA;
    static_assert(DMA == (BMODE == LOAD_DMA), "LOAD_DMA loads both operands");
    static_assert(!DMA || dma_tile<T>, "LOAD_DMA tile shape");
    static_assert(!DMA || 2 * T::D_STAGE * sizeof(float) <= 160 * 1024, "two DMA stages in LDS");
    __shared__ __attribute__((aligned(16)))
    float smem[2 * (DMA && T::D_STAGE > T::STAGE ? T::D_STAGE : T::STAGE)];

    const int tid = threadIdx.x;
    const int tiles_m = (g.M + T::BM - 1) / T::BM;
    const int tiles_n = (g.N - g.n_begin + T::BN - 1) / T::BN;
    int local, split, tm, tn;
    block_pos(local, split);
    tile_of(g.tile_begin + local, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * T::BM, n0 = g.n_begin + tn * T::BN;
    // Classifier head: this tile's rows of the next layer's weights, loaded
    // before the K loop so that their latency hides behind it.
    constexpr bool HEAD = head_tile<T, AMODE, BMODE>;
    const bool head = HEAD && g.head_w != nullptr;
    float head_wr[2] = {0.f, 0.f};
    if constexpr (HEAD) {
        static_assert(T::BN * HEAD_MAX_N2 <= 2 * T::THREADS, "two head weights per thread");
        if (head) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int e = (int)threadIdx.x + u * T::THREADS;
                if (e < T::BN * g.head_n2)
                    head_wr[u] = g.head_w[(size_t)(n0 + e / g.head_n2) * g.head_n2 + e % g.head_n2];
            }
        }
    }
    // K is consumed in whole stages: when BK does not divide K, the ragged
    // part is the first stage of split 0, which starts kpad below k = 0 and
    // is loaded with guards (zeros below 0); every later stage is a whole BK
    // and the loop body keeps guard-free loads.  (The conv loaders have
    // K % BK == 0.)
    const int kpad = is_nhwc<BMODE> ? 0 : (T::BK - g.K % T::BK) % T::BK;
    const int kbeg = split * g.k_per_split - kpad;
    const int kend = min(g.K, kbeg + g.k_per_split);
    const int nk = kend > kbeg ? (kend - kbeg + T::BK - 1) / T::BK : 0;

    if constexpr (is_nhwc<BMODE>) {
        static_assert((T::BN * T::KQ) % T::THREADS == 0, "B pixel rows must split evenly");
    } else {
        static_assert(T::THREADS % (T::BN / 4) == 0 || (T::BN / 4) % T::THREADS == 0,
                      "B column mapping");
    }
    // Items past a stage's count (when THREADS does not divide it) are skipped
    // by whole waves.
    constexpr bool A_TAIL = T::A_TOTAL % T::THREADS != 0;
    constexpr bool AT_TAIL = T::A_T_TOTAL % T::THREADS != 0;
    constexpr bool B_TAIL = T::B_TOTAL % T::THREADS != 0;
    if constexpr (is_trans<AMODE>) {
        static_assert(T::THREADS % (T::BM / 4) == 0 || (T::BM / 4) % T::THREADS == 0,
                      "transposed A column mapping");
    }
    // One stage of operands in flight from global memory to LDS.
    struct StageRegs {
        float4 ra[is_trans<AMODE> ? 1 : T::A_ITEMS];
        float4 rat[is_trans<AMODE> ? T::A_T_ITEMS : 1][4];
        float4 rb[is_nhwc<BMODE> ? 1 : T::B_ITEMS][4];
        float4 rbn[is_nhwc<BMODE> ? T::BN_ITEMS : 1];
    };
    StageRegs R0;
    // LOAD_VEC B on the long-stage (non-EARLY) tiles: each item's element
    // offset of its first k row, advanced BK rows per loaded stage, in place
    // of a 64-bit multiply per load and stage (measured 1% faster at 4096^3;
    // the EARLY tiles keep the multiply, 7% faster there at 1024^3).  An
    // offset rather than a pointer: the ragged first stage starts below row 0.
    constexpr bool B_PTR = BMODE == LOAD_VEC && !T::EARLY;
    ptrdiff_t b_vec_off[B_PTR ? T::B_ITEMS : 1];
    if constexpr (B_PTR) {
#pragma unroll
        for (int i = 0; i < T::B_ITEMS; ++i) {
            const int q = tid + i * T::THREADS;
            const int nq = q % (T::BN / 4), kq = q / (T::BN / 4);
            b_vec_off[i] = (ptrdiff_t)(kbeg + 4 * kq) * g.ldb + n0 + 4 * nq;
        }
    }

    // ---- NHWC / NCHW4 conv: each thread's B items are fixed (pixel, k-quad)
    // pairs.  Pixel geometry and the k-quad's channel-quad offset are decoded
    // once; the stage's (kh, kw, c0) comes from the stage start (uniform: one
    // stage never crosses a (kh, kw) boundary).
    int px_base[is_nhwc<BMODE> ? T::BN_ITEMS : 1];
    int px_ih[is_nhwc<BMODE> ? T::BN_ITEMS : 1];
    int px_iw[is_nhwc<BMODE> ? T::BN_ITEMS : 1];
    if constexpr (is_nhwc<BMODE>) {
#pragma unroll
        for (int i = 0; i < T::BN_ITEMS; ++i) {
            const int q = tid + i * T::THREADS;
            const int pg = n0 + item_pixel<T, BMODE>(q);
            if (pg < g.N) {
                int img, oh, ow;
                if constexpr (is_pool<BMODE>) {
                    // column = ((img * PP + window) * 4 + 2 dy + dx)
                    img = pg / (4 * g.PP);
                    const int r = pg - img * 4 * g.PP, win = r >> 2, d = r & 3;
                    const int ph = win / g.PW;
                    oh = 2 * ph + (d >> 1);
                    ow = 2 * (win - ph * g.PW) + (d & 1);
                } else {
                    img = pg / g.P;
                    const int p = pg - img * g.P;
                    oh = p / g.OW;
                    ow = p - oh * g.OW;
                }
                px_ih[i] = oh * g.stride - g.pad;
                px_iw[i] = ow * g.stride - g.pad;
                px_base[i] = img * g.CHW + (px_ih[i] * g.W + px_iw[i]) * g.pxs +
                             item_kquad<T, BMODE>(q) * g.cqs;
            } else {
                px_ih[i] = -(1 << 28); // never in range
                px_iw[i] = 0;
                px_base[i] = 0;
            }
        }
    }

    // ---- conv: per-thread column geometry, fixed for the whole K loop ----
    // Column c of the thread's 4 columns is n0 + nq + c*(BN/4) (spread so a
    // wave's scalar loads touch consecutive pixels).
    int col_base[4], col_ih[4], col_iw[4];
    if constexpr (BMODE == LOAD_CONV) {
        static_assert(T::THREADS % (T::BN / 4) == 0, "conv columns must be fixed per thread");
        const int nq = tid % (T::BN / 4);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int pg = n0 + nq + c * (T::BN / 4);
            if (pg < g.N) {
                const int img = pg / g.P, p = pg - img * g.P;
                const int oh = p / g.OW, ow = p - oh * g.OW;
                col_ih[c] = oh * g.stride - g.pad;
                col_iw[c] = ow * g.stride - g.pad;
                col_base[c] = img * g.CHW + col_ih[c] * g.W + col_iw[c];
            } else {
                col_ih[c] = -(1 << 28); // never in range
                col_iw[c] = 0;
                col_base[c] = 0;
            }
        }
    }

    // FULL: the tile lies inside M x N and the stage is a whole BK inside
    // [0, K), so the row/column/k guards compile away (every stage of the
    // interior tiles but a ragged first one).
    // part_tag (LoadPart) picks the operands: both, or A or B alone (a
    // stage's loads split over two MFMA groups).  again: k0 is the stage
    // loaded last, read once more (the B row offsets step back a stage and
    // are not advanced).
    auto load_stage = [&](auto full_tag, int k0, StageRegs &R, auto part_tag, bool again = false) {
        constexpr bool FULL = decltype(full_tag)::value;
        constexpr bool LA = decltype(part_tag)::value != LOAD_B_ONLY;
        constexpr bool LB = decltype(part_tag)::value != LOAD_A_ONLY;
        float4 *ra = R.ra;
        auto &rat = R.rat;
        auto &rb = R.rb;
        float4 *rbn = R.rbn;
#pragma unroll
        for (int i = 0; i < (is_trans<AMODE> && LA ? T::A_T_ITEMS : 0); ++i) {
            // item (kq, mq): rows k0+4kq .. +3 of At, columns m0+4mq .. +3
            // (vector) or m0+mq+c*BM/4 (scalar, c = 0..3)
            const int q = tid + i * T::THREADS;
            if (AT_TAIL && q >= T::A_T_TOTAL) break;
            const int mq = q % (T::BM / 4), kq = q / (T::BM / 4);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int gk = k0 + 4 * kq + u;
                // gk is below 0 in a ragged first stage: the row is an offset
                // (it wraps) or an address computed as an integer, and a
                // pointer into A is formed only where the guard admits a load
                if constexpr (AMODE == LOAD_TVEC) {
                    const size_t row = (size_t)gk * g.lda;
                    const int gm = m0 + 4 * mq;
                    rat[i][u] = (FULL || (gm < g.M && gk >= 0 && gk < kend))
                                    ? *reinterpret_cast<const float4 *>(g.A + (row + gm))
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    const float *row = row_address(g.A, gk, g.lda);
                    float v[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int gm = m0 + mq + c * (T::BM / 4);
                        v[c] = (FULL || (gm < g.M && gk >= 0 && gk < kend)) ? row[gm] : 0.f;
                    }
                    rat[i][u] = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < (is_trans<AMODE> || !LA ? 0 : T::A_ITEMS); ++i) {
            const int q = tid + i * T::THREADS;
            if (A_TAIL && q >= T::A_TOTAL) break;
            const int kq = q % T::KQ, m = q / T::KQ;
            const int gm = m0 + m, gk = k0 + 4 * kq;
            const size_t src = (size_t)gm * g.lda + gk;
            if constexpr (AMODE == LOAD_VEC) {
                ra[i] = (FULL || (gm < g.M && gk >= 0 && gk < kend))
                            ? *reinterpret_cast<const float4 *>(g.A + src)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                const bool rv = FULL || gm < g.M;
                ra[i].x = (rv && (FULL || (gk + 0 >= 0 && gk + 0 < kend))) ? g.A[src + 0] : 0.f;
                ra[i].y = (rv && (FULL || (gk + 1 >= 0 && gk + 1 < kend))) ? g.A[src + 1] : 0.f;
                ra[i].z = (rv && (FULL || (gk + 2 >= 0 && gk + 2 < kend))) ? g.A[src + 2] : 0.f;
                ra[i].w = (rv && (FULL || (gk + 3 >= 0 && gk + 3 < kend))) ? g.A[src + 3] : 0.f;
            }
        }
        if constexpr (is_nhwc<BMODE> && LB) {
            // k0 .. k0+BK-1 share (kh, kw): channels c0 .. c0+BK-1.
            const int khw = k0 / g.Cin, c0 = k0 - khw * g.Cin;
            const int kh = khw / g.KW, kw = khw - kh * g.KW;
            const int koff = (kh * g.W + kw) * g.pxs + (c0 >> 2) * g.cqs;
#pragma unroll
            for (int i = 0; i < T::BN_ITEMS; ++i) {
                const int ih = px_ih[i] + kh, iw = px_iw[i] + kw;
                const bool in = (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W &&
                                (FULL || k0 < kend);
                // a padding pixel's offset is below 0: formed into a pointer
                // only when the pixel is in the image
                const size_t src = (size_t)(px_base[i] + koff);
                if constexpr (is_planes<BMODE>) {
                    rbn[i] = in ? make_float4(g.B[src], g.B[src + g.chs],
                                              g.B[src + 2 * (size_t)g.chs],
                                              g.B[src + 3 * (size_t)g.chs])
                                : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    rbn[i] = in ? *reinterpret_cast<const float4 *>(g.B + src)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < (is_nhwc<BMODE> || !LB ? 0 : T::B_ITEMS); ++i) {
            const int q = tid + i * T::THREADS;
            if (B_TAIL && q >= T::B_TOTAL) break;
            const int nq = q % (T::BN / 4), kq = q / (T::BN / 4);
            if constexpr (BMODE == LOAD_VEC) {
                const int gn = n0 + 4 * nq;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int gk = k0 + 4 * kq + u;
                    const ptrdiff_t back = again ? (ptrdiff_t)T::BK * g.ldb : 0;
                    // an offset (it wraps below 0 for the ragged first stage,
                    // where the guard keeps it from becoming a pointer)
                    const size_t src = B_PTR ? (size_t)(b_vec_off[i] - back + (ptrdiff_t)u * g.ldb)
                                             : (size_t)gk * g.ldb + gn;
                    rb[i][u] = (FULL || (gn < g.N && gk >= 0 && gk < kend))
                                   ? *reinterpret_cast<const float4 *>(g.B + src)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
                }
                if constexpr (B_PTR) b_vec_off[i] += again ? 0 : (ptrdiff_t)T::BK * g.ldb;
            } else if constexpr (BMODE == LOAD_SCALAR) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int gk = k0 + 4 * kq + u;
                    const float *row = row_address(g.B, gk, g.ldb);
                    float v[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int gn = n0 + nq + c * (T::BN / 4);
                        v[c] = (FULL || (gn < g.N && gk >= 0 && gk < kend)) ? row[gn] : 0.f;
                    }
                    rb[i][u] = make_float4(v[0], v[1], v[2], v[3]);
                }
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int gk = k0 + 4 * kq + u;
                    float v[4] = {0.f, 0.f, 0.f, 0.f};
                    if (FULL || (gk >= 0 && gk < kend)) {
                        const int2 e = g.ktab[gk];
                        const int kh = e.y >> 16, kw = e.y & 0xffff;
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const int ih = col_ih[c] + kh, iw = col_iw[c] + kw;
                            if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                                v[c] = g.B[(size_t)(col_base[c] + e.x)];
                        }
                    }
                    rb[i][u] = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
        }
    };

    auto store_stage = [&](float *As, float *Bs, const StageRegs &R) {
        const float4 *ra = R.ra;
        const auto &rat = R.rat;
        const auto &rb = R.rb;
        const float4 *rbn = R.rbn;
#pragma unroll
        for (int i = 0; i < (is_trans<AMODE> ? T::A_T_ITEMS : 0); ++i) {
            const int q = tid + i * T::THREADS;
            if (AT_TAIL && q >= T::A_T_TOTAL) break;
            const int mq = q % (T::BM / 4), kq = q / (T::BM / 4);
            float *plane = As + kq * T::A_PLANE;
            // rat[i][u] holds k row k0+4kq+u for 4 m; LDS wants, per m, the 4
            // k values as one chunk: a 4x4 transpose in registers.
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int m = (AMODE == LOAD_TVEC) ? 4 * mq + c : mq + c * (T::BM / 4);
                float4 col;
                col.x = rat[i][0][c];
                col.y = rat[i][1][c];
                col.z = rat[i][2][c];
                col.w = rat[i][3][c];
                *reinterpret_cast<float4 *>(plane + m * 4) = col;
            }
        }
#pragma unroll
        for (int i = 0; i < (is_trans<AMODE> ? 0 : T::A_ITEMS); ++i) {
            const int q = tid + i * T::THREADS;
            if (A_TAIL && q >= T::A_TOTAL) break;
            const int kq = q % T::KQ, m = q / T::KQ;
            *reinterpret_cast<float4 *>(As + kq * T::A_PLANE + m * 4) = ra[i];
        }
        if constexpr (is_nhwc<BMODE>) {
#pragma unroll
            for (int i = 0; i < T::BN_ITEMS; ++i) {
                const int q = tid + i * T::THREADS;
                const int kq = item_kquad<T, BMODE>(q), n = item_pixel<T, BMODE>(q);
                *reinterpret_cast<float4 *>(Bs + kq * T::B_PLANE + b_slot(n) * 4) = rbn[i];
            }
        }
#pragma unroll
        for (int i = 0; i < (is_nhwc<BMODE> ? 0 : T::B_ITEMS); ++i) {
            const int q = tid + i * T::THREADS;
            if (B_TAIL && q >= T::B_TOTAL) break;
            const int nq = q % (T::BN / 4), kq = q / (T::BN / 4);
            float *plane = Bs + kq * T::B_PLANE;
            // rb[i][u] holds row k0+4kq+u for 4 columns; LDS wants, per column,
            // the 4 k values as one chunk: a 4x4 transpose in registers.
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int n = (BMODE == LOAD_VEC) ? 4 * nq + c : nq + c * (T::BN / 4);
                float4 col;
                col.x = rb[i][0][c];
                col.y = rb[i][1][c];
                col.z = rb[i][2][c];
                col.w = rb[i][3][c];
                *reinterpret_cast<float4 *>(plane + b_slot(n) * 4) = col;
            }
        }
    };

    const int wave = tid >> 6, lane = tid & 63;
    const int half = lane >> 5, r32 = lane & 31;
    const int wk = wave / (T::WM * T::WN), wsp = wave % (T::WM * T::WN);
    const int wm = wsp / T::WN, wn = wsp % T::WN;

    floatx16 acc[T::FM][T::FN];
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // Schedule of one stage kt (G = 8-k groups per wave):
    //   * the global loads of stage kt+1 are issued first (registers);
    //   * LDS operand reads run one 8-k group ahead of the MFMAs that use them,
    //     so each group's ds_read latency hides behind the previous group's
    //     MFMAs; they are spread one per two MFMAs over the head of the group
    //     (measured against issuing them together before it: 4096^3 1-2%,
    //     2048^3 1.5%, the config-4 conv 3.7% faster);
    //   * EARLY: halfway through, stage kt+1 is stored to the other LDS buffer
    //     (its last readers finished before the previous barrier), and the
    //     barrier comes before the last group's MFMAs, with the first reads of
    //     stage kt+1 issued right after it, so those MFMAs cover the read
    //     latency and the barrier costs little more than the waves' skew
    //     (measured faster for 64x64 and 128x128 tiles);
    //   * otherwise: stage kt+1 is stored to the other buffer right after the
    //     first group's MFMAs, and the barrier follows all G groups (measured
    //     faster for the 8-wave 256x256 tile, whose long stages already hide
    //     the barrier; storing after the first group rather than after the
    //     last keeps the stores' latency off the end of the stage: 4096^3
    //     134.4-136.9 -> 137.3-138.0 TFLOP/s, and after the second or third
    //     group was slower, 137.3 / 133.2).  With 16-byte A and B loads and
    //     at least 3 groups, the global loads run two stages ahead: stage
    //     kt+2's A rows go out among the MFMAs of group G-2 of stage kt and
    //     its B rows among those of group G-1, into the registers the store
    //     after group 0 has just emptied, instead of all at the top of
    //     stage kt+1 (4096^3 139.6 -> 142.0 TFLOP/s, 8192^3 141.0 -> 143.3;
    //     the loads in groups 1-2, or spaced 1 to 5 MFMAs apart, gained
    //     only 139.4-139.7).
    constexpr int GROUPS = T::BK / 8 / T::WK; // 8-k groups of this wave's k-group
    constexpr int STORE_AT = GROUPS / 2 - 1;   // store after this group's MFMAs
    // MFMAs between two of the next group's operand reads (the reads are
    // spread over the head of a group; all tiles have 4 FM FN >= 2 (FM + FN)).
    constexpr int READ_SPACING = 2;
    static_assert(4 * T::FM * T::FN >= READ_SPACING * (T::FM + T::FN), "read spacing");
    static_assert(GROUPS % 2 == 0, "operand registers alternate between even and odd groups");
    auto operand_bases = [&](int kt, const float *&a_base, const float *&b_base) {
        const float *As = smem + (kt & 1) * T::STAGE;
        const float *Bs = As + T::A_STAGE;
        a_base = As + (2 * GROUPS * wk + half) * T::A_PLANE + (wm * T::WTM + r32) * 4;
        b_base = Bs + (2 * GROUPS * wk + half) * T::B_PLANE + (wn * T::WTN + b_slot(r32)) * 4;
    };
    auto fetch = [&](const float *a_base, const float *b_base, int s8, float4 *fa, float4 *fb) {
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
            fa[i] = *reinterpret_cast<const float4 *>(a_base + 2 * s8 * T::A_PLANE + i * 128);
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
            fb[j] = *reinterpret_cast<const float4 *>(b_base + 2 * s8 * T::B_PLANE + j * 128);
    };
    auto mfma_group = [&](const float4 *fa, const float4 *fb) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int j = 0; j < T::FN; ++j)
                    acc[i][j] =
                        __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][t], fb[j][t], acc[i][j], 0, 0, 0);
    };
    auto lds_stage = [&](int kt) { return smem + (kt & 1) * T::STAGE; };

    auto main_loop = [&](auto full_tag) {
        if (nk <= 0) return;
        if (kbeg < 0)
            load_stage(std::false_type{}, kbeg, R0, load_ab); // the ragged first stage
        else
            load_stage(full_tag, kbeg, R0, load_ab);
        store_stage(smem, smem + T::A_STAGE, R0);
        __syncthreads();
        float4 fa[2][T::FM], fb[2][T::FN];
        const float *a_base, *b_base;
        if constexpr (!T::EARLY) {
            // AHEAD: loads two stages ahead, split over the last two groups
            constexpr bool AHEAD = AMODE == LOAD_VEC && BMODE == LOAD_VEC && GROUPS >= 3;
            constexpr int NMF = 4 * T::FM * T::FN, NRD = T::FM + T::FN;
            constexpr int NLA = T::A_ITEMS, NLB = 4 * T::B_ITEMS; // 16-byte loads
            // with loads ahead, reads and loads 3 MFMAs apart where they fit
            // (the 256x256 tile: 4096^3 +0.4%, 8192^3 +0.5% over 2)
            constexpr int SPACING = AHEAD && NMF >= 3 * (NRD + NLA) ? 3 : READ_SPACING;
            static_assert(!AHEAD || (NMF >= SPACING * (NRD + NLA) && NMF >= SPACING * NLB),
                          "loads two stages ahead fit among a group's MFMAs");
            if (AHEAD && nk > 1) load_stage(full_tag, kbeg + T::BK, R0, load_ab);
            for (int kt = 0; kt < nk; ++kt) {
                const bool more = kt + 1 < nk, more2 = kt + 2 < nk;
                if (!AHEAD && more) load_stage(full_tag, kbeg + (kt + 1) * T::BK, R0, load_ab);
                operand_bases(kt, a_base, b_base);
                fetch(a_base, b_base, 0, fa[0], fb[0]);
                __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);
#pragma unroll
                for (int s8 = 0; s8 < GROUPS; ++s8) {
                    const int cur = s8 & 1;
                    // the next group's operand reads go out one per
                    // SPACING MFMAs at the head of this group
                    if (s8 + 1 < GROUPS) fetch(a_base, b_base, s8 + 1, fa[cur ^ 1], fb[cur ^ 1]);
                    // Past the end the last stage is read again (in bounds,
                    // never stored): no branch splits the loop body.
                    const int k2 = kbeg + (more2 ? kt + 2 : nk - 1) * T::BK;
                    if (AHEAD && s8 == GROUPS - 2) load_stage(full_tag, k2, R0, load_a, !more2);
                    if (AHEAD && s8 == GROUPS - 1) load_stage(full_tag, k2, R0, load_b, !more2);
                    mfma_group(fa[cur], fb[cur]);
                    if (s8 + 1 < GROUPS) {
#pragma unroll
                        for (int r = 0; r < NRD; ++r) {
                            __builtin_amdgcn_sched_group_barrier(0x008, SPACING, 0);
                            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        }
                        if (AHEAD && s8 == GROUPS - 2) {
#pragma unroll
                            for (int r = 0; r < NLA; ++r) {
                                __builtin_amdgcn_sched_group_barrier(0x008, SPACING, 0);
                                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                            }
                            __builtin_amdgcn_sched_group_barrier(
                                0x008, NMF - SPACING * (NRD + NLA), 0);
                        } else {
                            __builtin_amdgcn_sched_group_barrier(0x008, NMF - SPACING * NRD, 0);
                        }
                    } else if (AHEAD) {
#pragma unroll
                        for (int r = 0; r < NLB; ++r) {
                            __builtin_amdgcn_sched_group_barrier(0x008, SPACING, 0);
                            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                        }
                        __builtin_amdgcn_sched_group_barrier(0x008, NMF - SPACING * NLB, 0);
                    } else {
                        __builtin_amdgcn_sched_group_barrier(0x008, NMF, 0);
                    }
                    // Unconditional: after the last stage this stores stale
                    // registers to the buffer the previous stage read, which
                    // no wave reads again (4096^3 +0.6%, 8192^3 +1.2% over
                    // a branch on kt + 1 < nk).
                    if (s8 == 0)
                        store_stage(lds_stage(kt + 1), lds_stage(kt + 1) + T::A_STAGE, R0);
                }
                __syncthreads();
            }
            return;
        }
        operand_bases(0, a_base, b_base);
        fetch(a_base, b_base, 0, fa[0], fb[0]);
        // Plain GEMM tiles (A and B row-major, 16-byte loads): with 32x32
        // wave tiles the next stage's loads go out after the first group's
        // operand reads rather than ahead of them (0.6% at 1024^3, 0.4 us of
        // the MLP's 47.7).  Plain and (pixel, k-quad) conv tiles with MFMAs to
        // spare spread the next stage's LDS stores one per MFMA over the
        // group after STORE_AT rather than issuing them together after it
        // (0.5% at 2048^3 and at the config-4 conv).
        constexpr bool PLAIN = AMODE == LOAD_VEC && BMODE == LOAD_VEC;
        constexpr bool PIXEL_B = AMODE == LOAD_VEC && is_nhwc<BMODE>;
        constexpr int NMF = 4 * T::FM * T::FN, NRD = T::FM + T::FN;
        // LDS stores per stage
        constexpr int NST = T::A_ITEMS + (PIXEL_B ? T::BN_ITEMS : 4 * T::B_ITEMS);
        constexpr bool LATE_LOADS = PLAIN && T::FM * T::FN == 1;
        constexpr bool SPREAD_STORES =
            (PLAIN || PIXEL_B) && GROUPS >= 4 && NMF - READ_SPACING * NRD >= NST;
        // Plain tiles run the loop body without branches: past the end the
        // last stage is loaded again (in bounds; a lone ragged stage takes
        // the guarded loop) and stored over the buffer the finished stage
        // read, and the next stage's first reads fetch values nothing uses
        // (1024^3 96.8 -> 99.8 TFLOP/s; the conv tiles measured 0.6% slower
        // so and keep the branches).
        constexpr bool NO_BRANCH = PLAIN;
        for (int kt = 0; kt < nk; ++kt) {
            const bool more = kt + 1 < nk;
            const int k1 = kbeg + (more ? kt + 1 : nk - 1) * T::BK;
            if (!LATE_LOADS && (NO_BRANCH || more)) load_stage(full_tag, k1, R0, load_ab);
#pragma unroll
            for (int s8 = 0; s8 + 1 < GROUPS; ++s8) {
                const int cur = s8 & 1;
                fetch(a_base, b_base, s8 + 1, fa[cur ^ 1], fb[cur ^ 1]);
                if (LATE_LOADS && s8 == 0 && (NO_BRANCH || more))
                    load_stage(full_tag, k1, R0, load_ab);
                const bool spread = SPREAD_STORES && s8 == STORE_AT + 1;
                if (spread && (NO_BRANCH || more))
                    store_stage(lds_stage(kt + 1), lds_stage(kt + 1) + T::A_STAGE, R0);
                mfma_group(fa[cur], fb[cur]);
                // The next group's LDS reads go out one per READ_SPACING MFMAs
                // at the head of this group (masks: 0x100 LDS read, 0x200 LDS
                // write, 0x8 MFMA).
#pragma unroll
                for (int r = 0; r < NRD; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, READ_SPACING, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                if (spread) {
#pragma unroll
                    for (int r = 0; r < NST; ++r) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                    }
                    __builtin_amdgcn_sched_group_barrier(0x008, NMF - READ_SPACING * NRD - NST, 0);
                } else {
                    __builtin_amdgcn_sched_group_barrier(0x008, NMF - READ_SPACING * NRD, 0);
                }
                if (!SPREAD_STORES && s8 == STORE_AT && (NO_BRANCH || more))
                    store_stage(lds_stage(kt + 1), lds_stage(kt + 1) + T::A_STAGE, R0);
            }
            __syncthreads();
            if (NO_BRANCH || more) {
                operand_bases(kt + 1, a_base, b_base);
                fetch(a_base, b_base, 0, fa[0], fb[0]);
                __builtin_amdgcn_sched_group_barrier(0x100, T::FM + T::FN, 0);
            }
            mfma_group(fa[1], fb[1]);
            __builtin_amdgcn_sched_group_barrier(0x008, 4 * T::FM * T::FN, 0);
        }
    };
    // ---- LOAD_DMA stage loop.  Per stage, wave w issues the DMAs of A row
    // quads (4 rows x 64 k: lane l takes row 4i + l / 16 and fills its slot
    // l % 16 with k-quad (l % 16 - row) & 15) and of B blocks b (4 k rows x
    // 64 columns: lane l takes row l / 16 and fills its slot l % 16 with
    // column chunk (l % 16 - 8 (b & 1)) & 15).  A stage
    // is in flight from the barrier of stage kt - 2 (before that stage's last
    // group, its buffer no longer read) to the barrier of stage kt - 1, whose
    // vmcnt(0) waits for it; the loop has no register staging and no LDS
    // stores.  A ragged first stage (k below 0) is loaded by the same lanes
    // with guarded 16-byte loads and stores to the same LDS places.
    auto dma_loop = [&](auto) {
        if (nk <= 0) return;
        constexpr int NW = T::THREADS / 64;
        constexpr int BP = T::BN / 64;                             // 64-column pieces per B block
        // DMAs per wave and stage (at least 1: this body is compiled for every tile)
        constexpr int DAI = T::BM / 4 / NW > 0 ? T::BM / 4 / NW : 1;
        constexpr int DBI = T::KQ * BP / NW > 0 ? T::KQ * BP / NW : 1;
        const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int du = lane >> 4, dc = lane & 15;
        size_t a_src[DAI], b_src[DBI]; // element offsets at k = 0
        int a_q[DAI];                  // the k-quad lane l fetches
#pragma unroll
        for (int j = 0; j < DAI; ++j) {
            const int r = 4 * (wv * DAI + j) + du;
            a_q[j] = (dc - r) & 15;
            a_src[j] = (size_t)(m0 + r) * g.lda + 4 * a_q[j];
        }
#pragma unroll
        for (int j = 0; j < DBI; ++j) {
            const int pc = wv * DBI + j, blk = pc / BP, h = pc - blk * BP;
            b_src[j] = (size_t)(4 * blk + du) * g.ldb + n0 + 64 * h + 4 * ((dc - 8 * (blk & 1)) & 15);
        }
        auto dma_stage = [&](int k0, int buf) {
            float *As = smem + buf * T::D_STAGE, *Bs = As + T::DA_STAGE;
#pragma unroll
            for (int j = 0; j < DAI; ++j)
                dma16(g.A + (a_src[j] + k0), As + (wv * DAI + j) * 4 * T::BK);
#pragma unroll
            for (int j = 0; j < DBI; ++j)
                dma16(g.B + (b_src[j] + (size_t)k0 * g.ldb), Bs + (wv * DBI + j) * 256);
        };
        auto guarded_stage = [&](int k0) { // buffer 0
            float *As = smem, *Bs = smem + T::DA_STAGE;
#pragma unroll
            for (int j = 0; j < DAI; ++j) {
                const int k = k0 + 4 * a_q[j];
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (k >= 0 && k < kend)
                    v = *reinterpret_cast<const float4 *>(g.A + (a_src[j] + (ptrdiff_t)k0));
                *reinterpret_cast<float4 *>(As + (wv * DAI + j) * 4 * T::BK + 4 * lane) = v;
            }
#pragma unroll
            for (int j = 0; j < DBI; ++j) {
                const int k = k0 + 4 * ((wv * DBI + j) / BP) + du;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (k >= 0 && k < kend)
                    v = *reinterpret_cast<const float4 *>(g.B + (b_src[j] + (ptrdiff_t)k0 * g.ldb));
                *reinterpret_cast<float4 *>(Bs + (wv * DBI + j) * 256 + 4 * lane) = v;
            }
        };
        // operand reads: group s8 of k-group wk, half-wave h takes k-quad
        // q = 2 GROUPS wk + 2 s8 + h (LOAD_VEC's order)
        int a_rd[GROUPS][T::FM];
#pragma unroll
        for (int s8 = 0; s8 < GROUPS; ++s8)
#pragma unroll
            for (int i = 0; i < T::FM; ++i) {
                const int r = wm * T::WTM + i * 32 + r32, q = 2 * GROUPS * wk + 2 * s8 + half;
                a_rd[s8][i] = r * T::BK + ((q + r) & 15) * 4;
            }
        int b_rd[T::FN]; // block parity = half
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int n = wn * T::WTN + j * 32 + r32, c = n & 63;
            b_rd[j] = (2 * GROUPS * wk + half) * T::DB_BLOCK + (n >> 6) * 256 +
                      (((c >> 2) + 8 * half) & 15) * 4 + (c & 3);
        }
        auto fetch_dma = [&](int buf, int s8, float4 *fa, float4 *fb) {
            const float *As = smem + buf * T::D_STAGE, *Bs = As + T::DA_STAGE;
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
                fa[i] = *reinterpret_cast<const float4 *>(As + a_rd[s8][i]);
#pragma unroll
            for (int j = 0; j < T::FN; ++j) {
                const float *b = Bs + b_rd[j] + 2 * s8 * T::DB_BLOCK;
                fb[j] = make_float4(b[0], b[64], b[128], b[192]);
            }
        };
        // LDS read instructions per group: A's 16-byte reads, B's 4 rows as
        // two ds_read2st64_b32
        constexpr int NMF = 4 * T::FM * T::FN, NRD = T::FM + 2 * T::FN;
        constexpr int SPACE = NMF >= 2 * NRD ? 2 : 1; // MFMAs before each operand read
        static_assert(NMF >= NRD, "one MFMA before each operand read");
        if (kbeg < 0)
            guarded_stage(kbeg);
        else
            dma_stage(kbeg, 0);
        if (nk > 1) dma_stage(kbeg + T::BK, 1);
        wait_vm();
        __syncthreads();
        float4 fa[2][T::FM], fb[2][T::FN];
        fetch_dma(0, 0, fa[0], fb[0]);
        for (int kt = 0; kt < nk; ++kt) {
            const int buf = kt & 1;
#pragma unroll
            for (int s8 = 0; s8 + 1 < GROUPS; ++s8) {
                const int cur = s8 & 1;
                fetch_dma(buf, s8 + 1, fa[cur ^ 1], fb[cur ^ 1]);
                mfma_group(fa[cur], fb[cur]);
#pragma unroll
                for (int r = 0; r < NRD; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, SPACE, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, NMF - SPACE * NRD, 0);
            }
            // waits for this wave's DMAs of stage kt + 1 (vmcnt) and its
            // reads of stage kt (lgkmcnt), then the barrier
            wait_vm();
            __syncthreads();
            if (kt + 2 < nk) dma_stage(kbeg + (kt + 2) * T::BK, buf);
            if (kt + 1 < nk) fetch_dma(buf ^ 1, 0, fa[0], fb[0]);
            mfma_group(fa[1], fb[1]);
        }
    };
    // The branch-free loop reads its last stage again past the end, unguarded
    // in a full tile, so that stage must be whole: a split whose only stage
    // is the ragged first one (K < BK) runs the guarded loop.
    if constexpr (DMA) {
        dma_loop(0);
    } else {
        const bool full_tile = m0 + T::BM <= g.M && (is_conv<BMODE> || n0 + T::BN <= g.N) &&
                               !(nk == 1 && kbeg < 0);
        if (full_tile)
            main_loop(std::true_type{});
        else
            main_loop(std::false_type{});
    }

    if constexpr (T::WK > 1) {
        // k-groups 1..WK-1 hand their sums to group 0 through LDS (free after
        // the loop's last barrier); group 0 adds them in group order.
        constexpr int PER_LANE = T::FM * T::FN * 4; // float4 per lane
        float4 *red = reinterpret_cast<float4 *>(smem);
        auto slot = [&](int grp, int i, int j, int q) {
            return ((((grp - 1) * T::WM * T::WN + wsp) * PER_LANE + (i * T::FN + j) * 4 + q) << 6) +
                   lane;
        };
        if (wk > 0) {
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int j = 0; j < T::FN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        red[slot(wk, i, j, q)] = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1],
                                                             acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
        }
        __syncthreads();
        if (wk > 0 && !head) return;
        for (int grp = 1; grp < (wk == 0 ? T::WK : 1); ++grp) {
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int j = 0; j < T::FN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 v = red[slot(grp, i, j, q)];
                        acc[i][j][4 * q + 0] += v.x;
                        acc[i][j][4 * q + 1] += v.y;
                        acc[i][j][4 * q + 2] += v.z;
                        acc[i][j][4 * q + 3] += v.w;
                    }
        }
    }

    if constexpr (HEAD) {
        if (head) {
            // Group 0 leaves the finished tile (bias, relu: the values the
            // store below would write) in LDS past the k-group sums; every
            // thread then forms (row, n) sums over the tile's 64 columns.
            constexpr int HS = T::BN + 1; // padded row of the tile
            static_assert(T::BM * T::BN + T::BM * HS + T::BN * HEAD_MAX_N2 <= 2 * T::STAGE,
                          "head tile and weights fit beside the k-group sums");
            float *ht = smem + T::BM * T::BN;
            float *hw = ht + T::BM * HS;
            const int n2 = g.head_n2;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int e = (int)threadIdx.x + u * T::THREADS;
                if (e < T::BN * n2) hw[(e / n2) * HEAD_MAX_N2 + e % n2] = head_wr[u];
            }
            if (wk == 0) {
                const bool hb = (g.flags & CAMEL_EPI_BIAS) != 0, hr = (g.flags & CAMEL_EPI_RELU) != 0;
                const int col = wn * T::WTN + r32;
                const float bc = hb ? g.bias[n0 + col] : 0.f;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int row = wm * T::WTM + 8 * (v >> 2) + 4 * half + (v & 3);
                    float x = acc[0][0][v];
                    if (hb) x = x + bc;
                    if (hr) x = relu_idiom(x);
                    ht[row * HS + col] = x;
                }
            }
            __syncthreads();
            // (Splitting each sum over a lane quad, 16 columns a lane, measured
            // slower: MLP forward 47.1 -> 49.2 us.)
            for (int o = (int)threadIdx.x; o < T::BM * n2; o += T::THREADS) {
                const int row = o / n2, n = o - row * n2;
                float s = 0.f;
#pragma unroll 16
                for (int j = 0; j < T::BN; ++j)
                    s = __builtin_fmaf(ht[row * HS + j], hw[j * HEAD_MAX_N2 + n], s);
                g.head_partial[((size_t)tn * g.M + m0 + row) * n2 + n] = s;
            }
            return;
        }
    }

    // ---- epilogue ----
    const bool has_bias = (g.flags & CAMEL_EPI_BIAS) != 0 && g.partial == nullptr;
    const bool has_relu = (g.flags & CAMEL_EPI_RELU) != 0 && g.partial == nullptr;
    // conv output in NCHW4 (the output rows of a lane's accumulator quad
    // v = 4u .. 4u+3 are 4 consecutive channels starting at a multiple of 4:
    // one 16-byte store per pixel)
    const bool q4 = is_conv<BMODE> && (g.flags & CAMEL_CONV_Y_NCHW4) != 0;
    // Bias values come into registers before the stores that follow them: as
    // far as the compiler knows C may alias bias, so a bias load after a
    // store waits for that store, one L2 round trip per element (measured:
    // 18% of a K = 288 conv).  Per-row (conv) biases are loaded per row block
    // i, 16 at a time; per-column (dense) biases once.
    float bcol[T::FN];
    if constexpr (!is_conv<BMODE>) {
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int col = n0 + wn * T::WTN + j * 32 + r32;
            bcol[j] = (has_bias && col < g.N) ? g.bias[col] : 0.f;
        }
    }
    auto row_bias = [&](int i, float *brow) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = m0 + wm * T::WTM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
            brow[v] = (has_bias && row < g.M) ? g.bias[row] : 0.f;
        }
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    // Calls body(bias_tag, relu_tag) with the epilogue flags as compile-time
    // types, so the element loops carry no uniform branches.
    auto with_flags = [&](auto body) {
        if (has_bias && has_relu)
            body(T_{}, T_{});
        else if (has_bias)
            body(T_{}, F_{});
        else if (has_relu)
            body(F_{}, T_{});
        else
            body(F_{}, F_{});
    };
    // Tiles inside M x N (most of them) store with no row / column guards.
    const bool full_out = g.partial == nullptr && m0 + T::BM <= g.M && n0 + T::BN <= g.N;
    if constexpr (is_pool<BMODE>) {
        if (full_out) {
            with_flags([&](auto bias_tag, auto relu_tag) {
#pragma unroll
                for (int i = 0; i < T::FM; ++i) {
                    float brow[16];
                    if constexpr (decltype(bias_tag)::value) row_bias(i, brow);
#pragma unroll
                    for (int j = 0; j < T::FN; ++j) {
                        const int col = n0 + wn * T::WTN + j * 32 + r32;
                        const int img = col / (4 * g.PP), win = (col - img * 4 * g.PP) >> 2;
                        float *out = g.C + (size_t)img * g.M * g.PP + win;
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const int row = m0 + wm * T::WTM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                            float x = acc[i][j][v];
                            if constexpr (decltype(bias_tag)::value) x = x + brow[v];
                            if constexpr (decltype(relu_tag)::value) x = relu_idiom(x);
                            const float x1 = quad_lane<1>(x), x2 = quad_lane<2>(x),
                                        x3 = quad_lane<3>(x);
                            float mx = x;
                            if (x1 > mx) mx = x1;
                            if (x2 > mx) mx = x2;
                            if (x3 > mx) mx = x3;
                            if ((r32 & 3) == 0) out[(size_t)row * g.PP] = mx;
                        }
                    }
                }
            });
            return;
        }
        if (g.partial == nullptr) {
            // A pool window is 4 consecutive columns, i.e. lanes r32 .. r32+3
            // of one half-wave (window starts are multiples of 4), one DPP
            // quad.  Every lane takes part in the moves; the window's first
            // lane stores the max in the order (0,0), (0,1), (1,0), (1,1) with
            // a strict '>' (maxpool2x2_kernel's rule).  Rows and columns past
            // the problem are uniform across a window.
#pragma unroll
            for (int i = 0; i < T::FM; ++i) {
                float brow[16];
                row_bias(i, brow);
#pragma unroll
                for (int j = 0; j < T::FN; ++j) {
                    const int col = n0 + wn * T::WTN + j * 32 + r32;
                    const int img = col / (4 * g.PP), win = (col - img * 4 * g.PP) >> 2;
                    const bool store_col = col < g.N && (r32 & 3) == 0;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int row = m0 + wm * T::WTM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                        float x = acc[i][j][v];
                        if (has_bias) x = x + brow[v];
                        if (has_relu) x = relu_idiom(x);
                        const float x1 = quad_lane<1>(x), x2 = quad_lane<2>(x), x3 = quad_lane<3>(x);
                        float mx = x;
                        if (x1 > mx) mx = x1;
                        if (x2 > mx) mx = x2;
                        if (x3 > mx) mx = x3;
                        if (store_col && row < g.M)
                            g.C[((size_t)img * g.M + row) * g.PP + win] = mx;
                    }
                }
            }
            return;
        }
    }
    if (full_out) {
        with_flags([&](auto bias_tag, auto relu_tag) {
#pragma unroll
            for (int i = 0; i < T::FM; ++i) {
                float brow[16];
                if constexpr (is_conv<BMODE> && decltype(bias_tag)::value) row_bias(i, brow);
#pragma unroll
                for (int j = 0; j < T::FN; ++j) {
                    const int col = n0 + wn * T::WTN + j * 32 + r32;
                    float *out;
                    if constexpr (is_conv<BMODE>) {
                        const int img = col / g.P, p = col - img * g.P;
                        out = g.C + (size_t)img * g.M * g.P + (q4 ? 4 * p : p);
                        if (q4) {
#pragma unroll
                            for (int u = 0; u < 4; ++u) {
                                const int row0 = m0 + wm * T::WTM + i * 32 + 8 * u + 4 * half;
                                float4 o;
#pragma unroll
                                for (int r = 0; r < 4; ++r) {
                                    float x = acc[i][j][4 * u + r];
                                    if constexpr (decltype(bias_tag)::value) x = x + brow[4 * u + r];
                                    if constexpr (decltype(relu_tag)::value) x = relu_idiom(x);
                                    o[r] = x;
                                }
                                *reinterpret_cast<float4 *>(out + (size_t)row0 * g.P) = o;
                            }
                            continue;
                        }
                    } else {
                        out = g.C + col;
                    }
                    const size_t row_stride = is_conv<BMODE> ? (size_t)g.P : (size_t)g.ldc;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int row = m0 + wm * T::WTM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                        float x = acc[i][j][v];
                        if constexpr (decltype(bias_tag)::value)
                            x = x + (is_conv<BMODE> ? brow[v] : bcol[j]);
                        if constexpr (decltype(relu_tag)::value) x = relu_idiom(x);
                        out[(size_t)row * row_stride] = x;
                    }
                }
            }
        });
        return;
    }
#pragma unroll
    for (int i = 0; i < T::FM; ++i) {
        float brow[16];
        if constexpr (is_conv<BMODE>) row_bias(i, brow);
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int col = n0 + wn * T::WTN + j * 32 + r32;
            if (col >= g.N) continue;
            size_t col_off = col;
            if constexpr (is_conv<BMODE>) {
                const int img = col / g.P, p = col - img * g.P;
                col_off = conv_out_off(g, q4, img, 0, p);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * T::WTM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                if (row >= g.M) continue;
                float x = acc[i][j][v];
                if (g.partial) {
                    g.partial[((size_t)split * gridDim.x + local) * (T::BM * T::BN) +
                              (size_t)(row - m0) * T::BN + (col - n0)] = x;
                    continue;
                }
                if constexpr (is_conv<BMODE>) {
                    if (has_bias) x = x + brow[v];
                } else {
                    if (has_bias) x = x + bcol[j];
                }
                if (has_relu) x = relu_idiom(x);
                if constexpr (is_conv<BMODE>)
                    g.C[col_off + (q4 ? (size_t)(row & ~3) * g.P + (row & 3) : (size_t)row * g.P)] = x;
                else
                    g.C[(size_t)row * g.ldc + col] = x;
            }
        }
    }
}

// Sums the K splits of tiles [tile_begin, tile_begin + ntiles) in split
// order (so results do not depend on scheduling), then bias and relu, and
// stores with the GEMM (row-major) or conv (NCHW or NCHW4) output mapping.
// POOL (pooled conv): one thread per pool window (4 consecutive columns of
// a tile), max of the 4 finished values in window order.
// sum_z partial[z * total + idx] for z = 0 .. splits-1, added in split order;
// loads go out up to 8 at a time (the guards are uniform) so their latencies
// overlap instead of each add waiting for its load.
__device__ __forceinline__ float sum_splits(const float *__restrict__ partial, size_t total,
                                            size_t idx, int splits) {
    float s = partial[idx];
    for (int z0 = 1; z0 < splits; z0 += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z0 + u < splits) t[u] = partial[(size_t)(z0 + u) * total + idx];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z0 + u < splits) s = s + t[u];
    }
    return s;
}

template <int BM, int BN, bool CONV, bool POOL = false>
__global__ __launch_bounds__(256) void tile_reduce_kernel(GemmArgs g, int ntiles, int splits) {
    const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N - g.n_begin + BN - 1) / BN;
    if constexpr (POOL) {
        const size_t per_tile = (size_t)BM * BN, total = (size_t)ntiles * per_tile;
        const size_t stride = (size_t)gridDim.x * blockDim.x;
        for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total / 4; q += stride) {
            const size_t idx = 4 * q;
            const int local = (int)(idx / per_tile);
            const int w = (int)(idx - (size_t)local * per_tile);
            int tm, tn;
            tile_of(g.tile_begin + local, tiles_m, tiles_n, tm, tn);
            const int row = tm * BM + w / BN, col = g.n_begin + tn * BN + w % BN;
            if (row >= g.M || col >= g.N) continue;
            float mx = 0.f;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                float s = sum_splits(g.partial, total, idx + d, splits);
                if (g.flags & CAMEL_EPI_BIAS) s = s + g.bias[row];
                if (g.flags & CAMEL_EPI_RELU) s = relu_idiom(s);
                if (d == 0 || s > mx) mx = s;
            }
            const int img = col / (4 * g.PP), win = (col - img * 4 * g.PP) >> 2;
            g.C[((size_t)img * g.M + row) * g.PP + win] = mx;
        }
        return;
    }
    const size_t per_tile = (size_t)BM * BN, total = (size_t)ntiles * per_tile;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
        const int local = (int)(idx / per_tile);
        const int w = (int)(idx - (size_t)local * per_tile);
        int tm, tn;
        tile_of(g.tile_begin + local, tiles_m, tiles_n, tm, tn);
        const int row = tm * BM + w / BN, col = g.n_begin + tn * BN + w % BN;
        if (row >= g.M || col >= g.N) continue;
        float s = sum_splits(g.partial, total, idx, splits);
        if (g.flags & CAMEL_EPI_BIAS) s = s + (CONV ? g.bias[row] : g.bias[col]);
        if (g.flags & CAMEL_EPI_RELU) s = relu_idiom(s);
        if constexpr (CONV) {
            const int img = col / g.P, p = col - img * g.P;
            g.C[conv_out_off(g, (g.flags & CAMEL_CONV_Y_NCHW4) != 0, img, row, p)] = s;
        } else {
            g.C[(size_t)row * g.ldc + col] = s;
        }
    }
}

// Thin GEMM (N <= 32, e.g. a classifier layer 1024 -> 10): too few columns
// for an MFMA tile to be useful.  B [K, N] is staged in LDS zero-padded to
// [256 * KV][NT] (NT >= N), so the inner loops run without guards; rows are
// STRIDE = NT + 4 floats apart so that the eight lanes one 16-byte LDS read
// serves per cycle land on disjoint banks.  Lanes take k = l + 64 i of a row
// of A (coalesced loads, zero past K) and accumulate all NT columns in fp32
// FMA; bias and relu as in the MFMA epilogue.  SOFTMAX (the fused
// dense..softmax of a classifier) then takes the row softmax across the
// wave's lanes, lane c holding column c, before the store.
//   * N <= 16 (sgemm_thin_rows_kernel): 16-wave work-groups own 4 rows, and
//     the 4 waves of a row take a quarter of the staged K each, so a CU
//     holds 16 waves and B is staged with one batch of loads per thread.  A
//     wave's 64 x NT partials meet in LDS (lane (c, s) adds the s-th segment
//     of column c, then a shuffle tree over the segments), and the row's
//     4 quarter sums are added in quarter order.  (One wave per row with a
//     64-lane shuffle tree per column took 9.1 us at 1024 x 1024 -> 10 with
//     the softmax; this takes 4.8 us.)
//   * 16 < N <= 32 (sgemm_thin_kernel): one wave per row over all of K and a
//     wave-shuffle tree per column (the 64 x 32 partials of 16 waves would
//     not fit in LDS beside B).
constexpr int THIN_LDS_FLOATS = 20480; // 80 KiB of B per work-group

template <int NT, int KV, bool SOFTMAX = false>
__global__ __launch_bounds__(256) void sgemm_thin_kernel(const float *__restrict__ A,
                                                         const float *__restrict__ B,
                                                         float *__restrict__ C, int M, int N, int K,
                                                         const float *__restrict__ bias, int flags) {
    constexpr int STRIDE = NT + 4, ROWS = 256 * KV, KPL = ROWS / 64; // k per lane
    static_assert(NT % 8 == 0 && ROWS * STRIDE <= THIN_LDS_FLOATS, "thin tile exceeds LDS");
    __shared__ __attribute__((aligned(16))) float bs[ROWS * STRIDE];
    const int lane = threadIdx.x & 63;
    const int waves = gridDim.x * (blockDim.x >> 6);
    auto load_row = [&](int m, float *av) {
        const float *a = A + (size_t)m * K;
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
            const int k = lane + 64 * i;
            av[i] = k < K ? a[k] : 0.f;
        }
    };
    int m = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    float av[KPL];
    // The first row's loads are in flight while B is staged (one batch of
    // loads per thread, then the LDS stores).
    if (m < M) load_row(m, av);
    constexpr int PER_THREAD = ROWS * NT / 256, BATCH = PER_THREAD < 32 ? PER_THREAD : 32;
    for (int base = 0; base < PER_THREAD; base += BATCH) {
        float v[BATCH];
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const int slot = (base + u) * 256 + (int)threadIdx.x;
            const int k = slot / NT, n = slot % NT;
            v[u] = (k < K && n < N) ? B[(size_t)k * N + n] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const int slot = (base + u) * 256 + (int)threadIdx.x;
            bs[(slot / NT) * STRIDE + slot % NT] = v[u];
        }
    }
    __syncthreads();
    for (; m < M; m += waves) {
        float acc[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[n] = 0.f;
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
            const float x = av[i];
            const float4 *brow = reinterpret_cast<const float4 *>(bs + (lane + 64 * i) * STRIDE);
#pragma unroll
            for (int q = 0; q < NT / 4; ++q) {
                const float4 bv = brow[q];
                acc[4 * q + 0] = __builtin_fmaf(x, bv.x, acc[4 * q + 0]);
                acc[4 * q + 1] = __builtin_fmaf(x, bv.y, acc[4 * q + 1]);
                acc[4 * q + 2] = __builtin_fmaf(x, bv.z, acc[4 * q + 2]);
                acc[4 * q + 3] = __builtin_fmaf(x, bv.w, acc[4 * q + 3]);
            }
        }
        // The next row's loads overlap this row's reduction.
        if (m + waves < M) load_row(m + waves, av);
        float out = 0.f;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            float v = acc[n];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            out = lane == n ? v : out;
        }
        if (lane < N) {
            if (flags & CAMEL_EPI_BIAS) out = out + bias[lane];
            if (flags & CAMEL_EPI_RELU) out = relu_idiom(out);
        }
        if constexpr (SOFTMAX) out = softmax_row_lanes(lane < N ? out : -INFINITY);
        if (lane < N) C[(size_t)m * N + lane] = out;
    }
}

// Row sources of the thin kernel's A operand: A[m][k] of a row-major matrix,
// or of the result of a split-K GEMM still in its partials, rebuilt the way
// tile_reduce_kernel finishes it (the splits added in split order, then the
// column bias and relu of that GEMM's epilogue), so a dense layer can feed
// the thin kernel without its reduce launch and with the same values.
struct RowsA {
    const float *A;
    int K;
    __device__ __forceinline__ float operator()(int m, int k) const { return A[(size_t)m * K + k]; }
};
struct SplitPartialsA {
    const float *partial; // [split][tile][BM * BN], tiles in tile_of order
    const float *bias;    // column bias of the GEMM (CAMEL_EPI_BIAS), or null
    int flags;            // that GEMM's epilogue flags
    int splits, ntiles, tiles_m, tiles_n, BM, BN;
    __device__ __forceinline__ float operator()(int m, int k) const {
        const int tm = m / BM, tn = k / BN;
        const size_t total = (size_t)ntiles * BM * BN;
        const size_t idx = (size_t)tile_id(tm, tn, tiles_m, tiles_n) * BM * BN +
                           (size_t)(m - tm * BM) * BN + (k - tn * BN);
        float v = sum_splits(partial, total, idx, splits);
        if (flags & CAMEL_EPI_BIAS) v = v + bias[k];
        if (flags & CAMEL_EPI_RELU) v = relu_idiom(v);
        return v;
    }
};

template <int NT, int KV, bool SOFTMAX = false, class ASrc = RowsA>
__global__ __launch_bounds__(1024) void sgemm_thin_rows_kernel(const ASrc src,
                                                               const float *__restrict__ B,
                                                               float *__restrict__ C, int M, int N,
                                                               int K, const float *__restrict__ bias,
                                                               int flags) {
    constexpr int STRIDE = NT + 4, ROWS = 256 * KV, KQ = ROWS / 4, RS = NT + 1;
    static_assert(NT == 8 || NT == 16, "partial segments assume 8 or 16 columns");
    __shared__ __attribute__((aligned(16))) float bs[ROWS * STRIDE];
    __shared__ float red[16][64 * RS]; // per wave: [lane][column], odd row stride
    __shared__ float quarter[4][4][NT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = wave >> 2, q = wave & 3; // row of the group, quarter of K
    const int groups = (M + 3) / 4;
    float av[KV];
    auto load_a = [&](int grp) {
        const int m = grp * 4 + r;
#pragma unroll
        for (int i = 0; i < KV; ++i) {
            const int k = q * KQ + lane + 64 * i;
            av[i] = (m < M && k < K) ? src(m, k) : 0.f;
        }
    };
    int grp = blockIdx.x;
    // The first group's A loads are in flight while B is staged (one batch of
    // loads per thread, then the LDS stores).
    load_a(grp);
    constexpr int PER_THREAD = ROWS * NT / 1024;
    float v[PER_THREAD];
#pragma unroll
    for (int u = 0; u < PER_THREAD; ++u) {
        const int slot = u * 1024 + (int)threadIdx.x;
        const int k = slot / NT, n = slot % NT;
        v[u] = (k < K && n < N) ? B[(size_t)k * N + n] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < PER_THREAD; ++u) {
        const int slot = u * 1024 + (int)threadIdx.x;
        bs[(slot / NT) * STRIDE + slot % NT] = v[u];
    }
    __syncthreads();
    float *rw = red[wave];
    const int c = lane % NT, seg = lane / NT; // 64 / NT segments of NT lanes
    for (; grp < groups; grp += gridDim.x) {
        float acc[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[n] = 0.f;
#pragma unroll
        for (int i = 0; i < KV; ++i) {
            const float x = av[i];
            const float4 *brow =
                reinterpret_cast<const float4 *>(bs + (q * KQ + lane + 64 * i) * STRIDE);
#pragma unroll
            for (int c4 = 0; c4 < NT / 4; ++c4) {
                const float4 bv = brow[c4];
                acc[4 * c4 + 0] = __builtin_fmaf(x, bv.x, acc[4 * c4 + 0]);
                acc[4 * c4 + 1] = __builtin_fmaf(x, bv.y, acc[4 * c4 + 1]);
                acc[4 * c4 + 2] = __builtin_fmaf(x, bv.z, acc[4 * c4 + 2]);
                acc[4 * c4 + 3] = __builtin_fmaf(x, bv.w, acc[4 * c4 + 3]);
            }
        }
        // The next group's loads overlap this group's reduction.
        if (grp + (int)gridDim.x < groups) load_a(grp + gridDim.x);
        // The wave's partials: lane (c, seg) adds lanes seg*NT .. seg*NT+NT-1
        // of column c (only this wave touches its slice, and a wave's LDS
        // operations run in order), then the segments meet by shuffles.
#pragma unroll
        for (int n = 0; n < NT; ++n) rw[lane * RS + n] = acc[n];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < NT; ++j) t += rw[(seg * NT + j) * RS + c];
#pragma unroll
        for (int off = NT; off < 64; off <<= 1) t += __shfl_xor(t, off);
        if (lane < NT) quarter[r][q][lane] = t;
        __syncthreads();
        const int m = grp * 4 + r;
        if (q == 0 && m < M) {
            float out = 0.f;
            if (lane < NT)
                out = ((quarter[r][0][lane] + quarter[r][1][lane]) + quarter[r][2][lane]) +
                      quarter[r][3][lane];
            if (lane < N) {
                if (flags & CAMEL_EPI_BIAS) out = out + bias[lane];
                if (flags & CAMEL_EPI_RELU) out = relu_idiom(out);
            }
            if constexpr (SOFTMAX) out = softmax_row_lanes(lane < N ? out : -INFINITY);
            if (lane < N) C[(size_t)m * N + lane] = out;
        }
        __syncthreads(); // quarter[] is rewritten by the next group
    }
}

// Finishes a classifier head run in a GEMM epilogue (GemmArgs::head_w): row
// m's N2 outputs are the tiles' partial sums added in tile order, then the
// second layer's bias and relu (and the row softmax), one wave per row, lane
// n holding column n -- the layout softmax_row_lanes takes.
template <bool SOFTMAX>
__global__ __launch_bounds__(256) void head_finish_kernel(const float *__restrict__ partial,
                                                          int tiles_n, int M, int N2,
                                                          const float *__restrict__ bias, int flags,
                                                          float *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return; // whole waves
    float out = 0.f;
    if (lane < N2) {
        const float *p = partial + (size_t)m * N2 + lane;
        const size_t tile_stride = (size_t)M * N2;
        float v[HEAD_MAX_N2];
#pragma unroll
        for (int t = 0; t < HEAD_MAX_N2; ++t) v[t] = t < tiles_n ? p[t * tile_stride] : 0.f;
#pragma unroll
        for (int t = 0; t < HEAD_MAX_N2; ++t)
            if (t < tiles_n) out = out + v[t];
        if (flags & CAMEL_EPI_BIAS) out = out + bias[lane];
        if (flags & CAMEL_EPI_RELU) out = relu_idiom(out);
    }
    if constexpr (SOFTMAX) out = softmax_row_lanes(lane < N2 ? out : -INFINITY);
    if (lane < N2) y[(size_t)m * N2 + lane] = out;
}

// True when the thin kernel serves C[M, N] = A[M, K] B[K, N].
bool thin_eligible(int64_t M, int64_t N, int64_t K) {
    if (N > 32 || N * 8 >= M) return false;
    // Longest k-slice per lane that the unrolled row loop holds in registers.
    return K <= (N <= 16 ? 1024 : 512);
}

// N <= 16 (and K <= 1024): the 16-wave kernel over rows from `src`.
template <bool SOFTMAX, class ASrc>
int launch_thin_rows(const ASrc &src, const float *B, float *C, int M, int N, int K,
                     const float *bias, int flags) {
    const int kv = std::max(1, (K + 255) / 256);
    // 4 rows per group, at most one work-group per CU (each stages B)
    const unsigned blocks = (unsigned)std::max<int64_t>(
        1, std::min<int64_t>(((int64_t)M + 3) / 4, device_cu_count()));
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(blocks), dim3(1024), 0, stream(), src, B, C, M, N, K, bias,
                           flags);
        return check_launch("sgemm_thin_rows_kernel");
    };
    if (N <= 8) {
        if (kv <= 1) return go(sgemm_thin_rows_kernel<8, 1, SOFTMAX, ASrc>);
        if (kv <= 2) return go(sgemm_thin_rows_kernel<8, 2, SOFTMAX, ASrc>);
        return go(sgemm_thin_rows_kernel<8, 4, SOFTMAX, ASrc>);
    }
    if (kv <= 1) return go(sgemm_thin_rows_kernel<16, 1, SOFTMAX, ASrc>);
    if (kv <= 2) return go(sgemm_thin_rows_kernel<16, 2, SOFTMAX, ASrc>);
    return go(sgemm_thin_rows_kernel<16, 4, SOFTMAX, ASrc>);
}

template <bool SOFTMAX = false>
int launch_thin(const float *A, const float *B, float *C, int M, int N, int K, const float *bias,
                int flags) {
    const int kv = std::max(1, (K + 255) / 256);
    if (N <= 16) return launch_thin_rows<SOFTMAX>(RowsA{A, K}, B, C, M, N, K, bias, flags);
    // Enough waves to cover the rows once, at most one work-group per CU
    // (each work-group stages all of B).
    const unsigned blocks = (unsigned)std::max<int64_t>(
        1, std::min<int64_t>((M + 3) / 4, device_cu_count()));
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), 0, stream(), A, B, C, M, N, K, bias,
                           flags);
        return check_launch("sgemm_thin_kernel");
    };
    if (kv <= 1) return go(sgemm_thin_kernel<32, 1, SOFTMAX>);
    return go(sgemm_thin_kernel<32, 2, SOFTMAX>);
}

// Skinny GEMM (M <= 32, e.g. M = 16, N = K = 4096): B is read once from HBM
// and dominates the traffic, so the kernel is a streaming pass over B.
//   * a work-group owns 64 columns x SK_CHUNK * CH k; its 8 waves take
//     interleaved chunks (wave w, chunk c: rows kb0 + (8 c + w) * 16 .. +15),
//     so at any time the work-group reads one contiguous block of rows;
//   * within a chunk lane l takes rows base + 4 (l / 16) + s (s = 0..3) and
//     one 16-byte piece of each, columns n0 + 4 (l % 16) .. +3: one load
//     instruction covers 4 rows x 256 contiguous bytes;
//   * v_mfma_f32_16x16x4_f32 takes A[i][k] from lane i + 16 k and B[k][j]
//     from lane j + 16 k; the 4 floats of a lane's piece feed 4 MFMAs whose
//     column j stands for column n0 + 4 j + c (c = 0..3), so no shuffle is
//     needed; the accumulator of MFMA c holds rows 4 (l / 16) + v at column
//     n0 + 4 (l % 16) + c.  Lane l's 4 k of a chunk are contiguous, so its A
//     values are one 16-byte load (A is small and stays in L2);
//   * B is read with nontemporal loads (it is read once; they measured 7%
//     faster than cached ones), a chunk's 4 loads issued together and
//     multiplied once they land -- a register double buffer that kept the
//     next chunk in flight measured 2% slower (the 8 waves of a CU already
//     overlap one another's loads); scheduling barriers keep the compiler
//     from interleaving a chunk's loads with its MFMAs.  Chunks of 4 rows
//     per lane rather than 8 halve the last chunk's MFMAs, which no load
//     overlaps (16 x 4096 x 4096: 16.07 -> 15.31 us per call);
//   * the 8 waves' sums meet in LDS in wave order; thread x then owns row
//     x / 16 and 4 consecutive columns, so the results (or the partials of
//     work-groups along K, [ks][M][N], which skinny_reduce_kernel sums in ks
//     order before the epilogue) leave as one 16-byte store per thread.
//     Letting the last work-group of a strip add the partials needs
//     device-scope release/acquire fences, and on this chip each one writes
//     back or invalidates an XCD's whole L2: measured several times slower.
// Work-groups whose rows, columns or k run past the operands take the same
// loop with guarded scalar loads (a guarded load compiles to a branch, after
// which the compiler waits for all loads at once, so full work-groups keep
// the guard-free path).
constexpr int SK_WAVES = 8;
constexpr int SK_COLS = 64;
constexpr int SK_STEPS = 4;                          // 4-row MFMA steps per chunk and wave
constexpr int SK_CHUNK = SK_WAVES * 4 * SK_STEPS;    // k rows per chunk of the work-group
constexpr int SK_MAX_KGROUPS = 65535;                // grid.y limit

template <int MT, int CH>
__global__ __launch_bounds__(SK_WAVES * 64) void sgemm_skinny_kernel(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int M, int N,
    int K, const float *__restrict__ bias, int flags, float *__restrict__ partial, int a_vec) {
    typedef float floatx4 __attribute__((ext_vector_type(4)));
    constexpr int S = SK_STEPS, KR = SK_CHUNK * CH;
    __shared__ float4 red[SK_WAVES][MT * 4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q = lane >> 4;
    const int strip = blockIdx.x, ks = blockIdx.y, nks = gridDim.y;
    const int n0 = strip * SK_COLS;
    const int kb0 = ks * KR;
    const int krow0 = kb0 + wave * 4 * S + q * S; // lane's first k of chunk 0
    const int col = n0 + 4 * r16;

    floatx4 acc[MT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[t][c] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto stream_k = [&](auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
        floatx4 b[S];
        float4 a[MT][S / 4];
        auto load = [&](int c) {
            const int kc = krow0 + c * SK_CHUNK;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int row = 16 * t + r16;
#pragma unroll
                for (int j = 0; j < S / 4; ++j) {
                    const int k = kc + 4 * j;
                    if (FULL) {
                        a[t][j] = *reinterpret_cast<const float4 *>(A + (size_t)row * K + k);
                    } else {
                        float e[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            e[i] = (row < M && k + i < K) ? A[(size_t)row * K + k + i] : 0.f;
                        a[t][j] = make_float4(e[0], e[1], e[2], e[3]);
                    }
                }
            }
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int k = kc + s;
                b[s] = (FULL || (col < N && k < K))
                           ? __builtin_nontemporal_load(
                                 reinterpret_cast<const floatx4 *>(B + (size_t)k * N + col))
                           : floatx4{0.f, 0.f, 0.f, 0.f};
            }
        };
        auto multiply = [&]() {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const float4 a4 = a[t][s / 4];
                    const float av = (s % 4 == 0) ? a4.x : (s % 4 == 1) ? a4.y : (s % 4 == 2) ? a4.z : a4.w;
                    acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b[s][0], acc[t][0], 0, 0, 0);
                    acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b[s][1], acc[t][1], 0, 0, 0);
                    acc[t][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b[s][2], acc[t][2], 0, 0, 0);
                    acc[t][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b[s][3], acc[t][3], 0, 0, 0);
                }
        };
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            load(c);
            __builtin_amdgcn_sched_barrier(0);
            multiply();
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if (a_vec && n0 + SK_COLS <= N && kb0 + KR <= K)
        stream_k(std::true_type{});
    else
        stream_k(std::false_type{});

#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c)
            red[wave][t * 4 + c][lane] = make_float4(acc[t][c][0], acc[t][c][1], acc[t][c][2],
                                                     acc[t][c][3]);
    __syncthreads();

    // Thread x < MT*256 owns row x / 16 and columns n0 + 4 (x % 16) .. +3.
    // Row r = 16 t + 4 g + v sits in element v of accumulator (t, c) of lane
    // 16 g + x % 16, for column n0 + 4 (x % 16) + c.
    const int x = threadIdx.x;
    if (x >= MT * 256) return;
    const int row = x >> 4, cg = x & 15;
    const int ocol = n0 + 4 * cg;
    if (row >= M || ocol >= N) return; // N % 4 == 0: a column group is all in or all out
    const int t = row >> 4, sl = ((row & 15) >> 2) * 16 + cg, e = row & 3;
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < SK_WAVES; ++w) s += reinterpret_cast<const float *>(&red[w][t * 4 + c][sl])[e];
        v[c] = s;
    }
    if (nks == 1) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float y = v[c];
            if (flags & CAMEL_EPI_BIAS) y = y + bias[ocol + c];
            if (flags & CAMEL_EPI_RELU) y = relu_idiom(y);
            v[c] = y;
        }
        *reinterpret_cast<float4 *>(C + (size_t)row * N + ocol) = make_float4(v[0], v[1], v[2], v[3]);
        return;
    }
    // partial layout [ks][M][N]
    *reinterpret_cast<float4 *>(partial + ((size_t)ks * M + row) * N + ocol) =
        make_float4(v[0], v[1], v[2], v[3]);
}

// Sums the skinny kernel's k partials in ks order, then bias and relu; one
// thread per 4 consecutive outputs of a row (N % 4 == 0).  Small work-groups
// (SK_REDUCE_THREADS) spread the few outputs over many CUs; the partials are
// read once, with nontemporal loads.  With `strips` > 0 (N a multiple of
// SK_COLS), work-group b takes 4 rows of strip b % strips: the skinny
// kernel's work-groups of that strip (block ids strip + strips * ks) ran on
// the same XCD when strips % 8 == 0, so the partials are read from that
// XCD's L2 (16 x 4096 x 4096: 15.30 -> 15.03 us per call); otherwise one
// thread per float4 in row-major order.
constexpr int SK_REDUCE_THREADS = 64;
static_assert(SK_REDUCE_THREADS == 4 * SK_COLS / 4, "a strip-mapped work-group is 4 rows of a strip");

__global__ __launch_bounds__(SK_REDUCE_THREADS) void skinny_reduce_kernel(
    const float4 *__restrict__ partial, float4 *__restrict__ C, int M, int N, int nks,
    const float *__restrict__ bias, int flags, int strips) {
    typedef float floatx4 __attribute__((ext_vector_type(4)));
    const size_t total4 = (size_t)M * N / 4;
    size_t idx;
    if (strips > 0) {
        const int strip = blockIdx.x % strips, rows4 = blockIdx.x / strips;
        const int row = 4 * rows4 + threadIdx.x / (SK_COLS / 4);
        if (row >= M) return;
        idx = ((size_t)row * N + (size_t)strip * SK_COLS) / 4 + threadIdx.x % (SK_COLS / 4);
    } else {
        idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
        if (idx >= total4) return;
    }
    const floatx4 *p4 = reinterpret_cast<const floatx4 *>(partial);
    // k groups added in order; their loads go out up to 8 at a time
    const floatx4 y0 = __builtin_nontemporal_load(p4 + idx);
    float4 y = make_float4(y0[0], y0[1], y0[2], y0[3]);
    for (int z0 = 1; z0 < nks; z0 += 8) {
        floatx4 p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z0 + u < nks) p[u] = __builtin_nontemporal_load(p4 + (size_t)(z0 + u) * total4 + idx);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (z0 + u < nks) {
                y.x = y.x + p[u][0];
                y.y = y.y + p[u][1];
                y.z = y.z + p[u][2];
                y.w = y.w + p[u][3];
            }
        }
    }
    if (flags & CAMEL_EPI_BIAS) {
        const size_t col = (idx * 4) % (size_t)N;
        y.x = y.x + bias[col];
        y.y = y.y + bias[col + 1];
        y.z = y.z + bias[col + 2];
        y.w = y.w + bias[col + 3];
    }
    if (flags & CAMEL_EPI_RELU) {
        y.x = relu_idiom(y.x);
        y.y = relu_idiom(y.y);
        y.z = relu_idiom(y.z);
        y.w = relu_idiom(y.w);
    }
    C[idx] = y;
}

// Mixed-dtype matmul: one thread per output, double accumulation in k order
// exactly as operators.cpp:757-766, rounded through setFromDouble.
__global__ void matmul_generic_kernel(int adt, const void *A, int bdt, const void *B, int odt,
                                      void *C, int64_t M, int64_t N, int64_t K) {
    const int64_t total = M * N;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
        const int64_t i = idx / N, j = idx % N;
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k)
            acc += load_as_double(adt, A, i * K + k) * load_as_double(bdt, B, k * N + j);
        store_from_double(odt, C, idx, acc);
    }
}

// ---- conv helpers ----------------------------------------------------------------

// x [N][C][HW] -> xt [N][HW][C] through LDS, one image per grid z; the
// extra z slice (z == N) reorders the weights w [Co][C][KHW] -> wt [Co][KHW][C]
// (K ordered (kh, kw, c)) in the same launch.
//   VEC (HW % 4 == 0, C % 4 == 0, 16-byte aligned): tiles of 32 channels x
//   TP_VEC pixels, 16-byte global loads along pixels and 16-byte stores along
//   channels, 4 of each per thread;
//   otherwise 32 x 32 tiles of 4-byte accesses.
constexpr int TP_VEC = 128;

__device__ __forceinline__ void reorder_weights(const float *__restrict__ w, float *__restrict__ wt,
                                                int Co, int C, int KHW) {
    const int total = Co * C * KHW;
    const int nthreads = gridDim.x * gridDim.y * blockDim.x;
    for (int i = (blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += nthreads) {
        const int co = i / (C * KHW), r = i - co * C * KHW;
        const int c = r / KHW, khw = r - c * KHW;
        wt[(size_t)co * C * KHW + (size_t)khw * C + c] = w[i];
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void nchw_to_nhwc_kernel(const float *__restrict__ x,
                                                           float *__restrict__ xt, int C, int HW,
                                                           const float *__restrict__ w,
                                                           float *__restrict__ wt, int Co,
                                                           int KHW) {
    constexpr int TP = VEC ? TP_VEC : 32, LD = TP + 1;
    __shared__ float tile[32 * LD];
    if (blockIdx.z == gridDim.z - 1) {
        reorder_weights(w, wt, Co, C, KHW);
        return;
    }
    const size_t img = blockIdx.z;
    const float *src = x + img * (size_t)C * HW;
    float *dst = xt + img * (size_t)C * HW;
    const int p0 = blockIdx.x * TP, c0 = blockIdx.y * 32;
    if constexpr (VEC) {
        // load: item i -> channel c0 + i / (TP/4), pixels p0 + 4 (i % (TP/4)) .. +3
#pragma unroll
        for (int u = 0; u < 32 * TP / 4 / 256; ++u) {
            const int i = threadIdx.x + 256 * u;
            const int c = i / (TP / 4), p = 4 * (i % (TP / 4));
            if (c0 + c < C && p0 + p < HW) {
                const float4 v =
                    *reinterpret_cast<const float4 *>(src + (size_t)(c0 + c) * HW + p0 + p);
                tile[c * LD + p] = v.x;
                tile[c * LD + p + 1] = v.y;
                tile[c * LD + p + 2] = v.z;
                tile[c * LD + p + 3] = v.w;
            }
        }
        __syncthreads();
        // store: item i -> pixel p0 + i / 8, channels c0 + 4 (i % 8) .. +3
#pragma unroll
        for (int u = 0; u < 32 * TP / 4 / 256; ++u) {
            const int i = threadIdx.x + 256 * u;
            const int p = i / 8, c = 4 * (i % 8);
            if (p0 + p < HW && c0 + c < C) {
                const float4 v = make_float4(tile[c * LD + p], tile[(c + 1) * LD + p],
                                             tile[(c + 2) * LD + p], tile[(c + 3) * LD + p]);
                *reinterpret_cast<float4 *>(dst + (size_t)(p0 + p) * C + c0 + c) = v;
            }
        }
    } else {
        const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
        for (int k = ty; k < 32; k += 8) {
            const int c = c0 + k, p = p0 + tx;
            if (c < C && p < HW) tile[k * LD + tx] = src[(size_t)c * HW + p];
        }
        __syncthreads();
#pragma unroll
        for (int k = ty; k < 32; k += 8) {
            const int p = p0 + k, c = c0 + tx;
            if (c < C && p < HW) dst[(size_t)p * C + c] = tile[tx * LD + k];
        }
    }
}

// NCHW <-> NCHW4 ([N][C/4][H][W][4], C % 4 == 0) over `quads` = N*C/4
// channel quads of HW pixels.  Thread = (channel quad, pixel): on the NCHW
// side four scalar accesses one plane apart (each coalesced over a wave's
// consecutive pixels), on the NCHW4 side one 16-byte access.
template <bool TO_Q4>
__global__ __launch_bounds__(256) void quad_layout_kernel(const float *__restrict__ src,
                                                          float *__restrict__ dst, int64_t quads,
                                                          int HW) {
    const int64_t total = quads * HW, step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        const int64_t q = i / HW;
        const size_t plane = (size_t)(4 * q) * HW + (size_t)(i - q * HW);
        if constexpr (TO_Q4) {
            reinterpret_cast<float4 *>(dst)[i] =
                make_float4(src[plane], src[plane + HW], src[plane + 2 * (size_t)HW],
                            src[plane + 3 * (size_t)HW]);
        } else {
            const float4 v = reinterpret_cast<const float4 *>(src)[i];
            dst[plane] = v.x;
            dst[plane + HW] = v.y;
            dst[plane + 2 * (size_t)HW] = v.z;
            dst[plane + 3 * (size_t)HW] = v.w;
        }
    }
}

// Direct convolution for a tiny reduction (C*KH*KW <= DIRECT_MAX_K, e.g. the
// first layer of an image CNN with C = 1): one thread per output pixel, all
// output channels.  The patch is loaded once into registers; the weights are
// wave-uniform and come in through scalar loads, so each output channel is
// KH*KW*C FMAs with a scalar operand, and the kernel runs at the speed of
// its output stores.  Accumulation runs in k = (c, kh, kw) ascending order
// with fp32 FMA, the same order as the GEMM path; bias then relu as
// x * (x > 0).
constexpr int DIRECT_MAX_K = 32;

// KMAX >= C*KH*KW: the k loops unroll over KMAX so the patch stays in
// registers.  EXACT (KMAX == C*KH*KW): no per-k guard, so the weight loads of
// a channel batch into a few scalar loads (a guarded one becomes a branch
// around a lone scalar load and its full latency).
// PIX consecutive output pixels per thread (P % PIX == 0, so they share an
// image): the channel loop then stores PIX-wide vectors.
// Q4: y is NCHW4 ([N][Co/4][OH][OW][4], Co % 4 == 0, 16-byte aligned); the
// channel loop runs a channel quad at a time and stores one 16-byte vector
// per pixel, consecutive lanes on consecutive pixels (the same values as the
// NCHW variant: each output is the same FMA chain).
template <int KMAX, bool EXACT, int PIX, bool Q4 = false>
__global__ __launch_bounds__(256) void conv2d_direct_kernel(
    const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    float *__restrict__ y, int NP, int P, int OW, int C, int H, int W, int Co, int KH, int KW,
    int stride, int pad, int flags) {
    typedef float vecp __attribute__((ext_vector_type(PIX)));
    const int K = C * KH * KW;
    const int pg = (blockIdx.x * blockDim.x + threadIdx.x) * PIX;
    if (pg >= NP) return;
    const int img = pg / P, p = pg - img * P;
    const float *xi = x + (size_t)img * C * H * W;
    float xv[PIX][KMAX];
#pragma unroll
    for (int j = 0; j < PIX; ++j) {
        const int oh = (p + j) / OW, ow = (p + j) - oh * OW;
        const int ih0 = oh * stride - pad, iw0 = ow * stride - pad;
        int c = 0, kh = 0, kw = 0;
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
            float v = 0.f;
            if (EXACT || k < K) {
                const int ih = ih0 + kh, iw = iw0 + kw;
                if ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W)
                    v = xi[(size_t)c * H * W + (size_t)ih * W + iw];
                if (++kw == KW) {
                    kw = 0;
                    if (++kh == KH) {
                        kh = 0;
                        ++c;
                    }
                }
            }
            xv[j][k] = v;
        }
    }
    float *yo = y + (size_t)img * Co * P + (Q4 ? 4 * (size_t)p : p);
    // Epilogue flags are fixed per variant so the channel loop has no
    // branches and its scalar loads batch across unrolled channels.
    auto channels = [&](auto has_bias, auto has_relu) {
        if constexpr (Q4) {
            for (int co = 0; co < Co; co += 4) {
                float4 out[PIX];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float *wr = w + (size_t)(co + r) * K;
#pragma unroll
                    for (int j = 0; j < PIX; ++j) {
                        float acc = 0.f;
#pragma unroll
                        for (int k = 0; k < KMAX; ++k)
                            if (EXACT || k < K) acc = __builtin_fmaf(wr[k], xv[j][k], acc);
                        if constexpr (decltype(has_bias)::value) acc = acc + bias[co + r];
                        if constexpr (decltype(has_relu)::value) acc = relu_idiom(acc);
                        out[j][r] = acc;
                    }
                }
#pragma unroll
                for (int j = 0; j < PIX; ++j)
                    *reinterpret_cast<float4 *>(yo + (size_t)co * P + 4 * j) = out[j];
            }
            return;
        }
#pragma unroll 4
        for (int co = 0; co < Co; ++co) {
            const float *wr = w + (size_t)co * K;
            vecp out;
#pragma unroll
            for (int j = 0; j < PIX; ++j) {
                float acc = 0.f;
#pragma unroll
                for (int k = 0; k < KMAX; ++k)
                    if (EXACT || k < K) acc = __builtin_fmaf(wr[k], xv[j][k], acc);
                if constexpr (decltype(has_bias)::value) acc = acc + bias[co];
                if constexpr (decltype(has_relu)::value) acc = relu_idiom(acc);
                out[j] = acc;
            }
            *reinterpret_cast<vecp *>(yo + (size_t)co * P) = out;
        }
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    const bool b = (flags & CAMEL_EPI_BIAS) != 0, r = (flags & CAMEL_EPI_RELU) != 0;
    if (b && r)
        channels(T_{}, T_{});
    else if (b)
        channels(T_{}, F_{});
    else if (r)
        channels(F_{}, T_{});
    else
        channels(F_{}, F_{});
}

// Direct convolution writing NHWC y [N][OH][OW][Co] (Co % 4 == 0, 16-byte
// aligned), for a consumer that reads NHWC.  Thread = one output pixel of a
// block's 256 consecutive pixels, channels as in conv2d_direct_kernel (the
// same k-ascending fp32 FMA chain with wave-uniform weights through scalar
// loads, bias, relu, so both layouts hold identical values), DN_CH channels
// at a time through an LDS tile [pixel][channel]; the block then writes its
// 256 pixel rows with 16-byte stores, which for Co <= DN_CH is one
// contiguous run of 256 Co floats.  (Storing each thread's channels straight
// to NHWC puts a wave's 16-byte stores 64 lines apart, and a thread per
// (pixel, 4 channels) issues per-lane weight loads: both measured 3x slower
// than the NCHW kernel.)
constexpr int DN_PIX = 256, DN_CH = 32;

template <int KMAX, bool EXACT, int CH = DN_CH, int PIXB = DN_PIX>
__global__ __launch_bounds__(PIXB) void conv2d_direct_nhwc_kernel(
    const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    float *__restrict__ y, int NP, int P, int OW, int C, int H, int W, int Co, int KH, int KW,
    int stride, int pad, int flags) {
    constexpr int LD = CH + 1; // odd row stride: a wave's column writes hit distinct banks
    __shared__ float tile[PIXB * LD];
    const int K = C * KH * KW;
    const int pg0 = blockIdx.x * PIXB, pg = pg0 + (int)threadIdx.x;
    const int npix = min(PIXB, NP - pg0);
    float xv[KMAX];
    {
        const int pc = pg < NP ? pg : NP - 1; // rows past the end compute a copy, never stored
        const int img = pc / P, p = pc - img * P;
        const int oh = p / OW, ow = p - oh * OW;
        const int ih0 = oh * stride - pad, iw0 = ow * stride - pad;
        const float *xi = x + (size_t)img * C * H * W;
        int c = 0, kh = 0, kw = 0;
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
            float v = 0.f;
            if (EXACT || k < K) {
                const int ih = ih0 + kh, iw = iw0 + kw;
                if (ih >= 0 && ih < H && iw >= 0 && iw < W) v = xi[((size_t)c * H + ih) * W + iw];
                if (++kw == KW) {
                    kw = 0;
                    if (++kh == KH) {
                        kh = 0;
                        ++c;
                    }
                }
            }
            xv[k] = v;
        }
    }
    float *trow = tile + threadIdx.x * LD;
    auto channels = [&](auto has_bias, auto has_relu, int c0, int cw) {
#pragma unroll 4
        for (int cc = 0; cc < cw; ++cc) {
            const int co = c0 + cc;
            const float *wr = w + (size_t)co * K;
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < KMAX; ++k)
                if (EXACT || k < K) acc = __builtin_fmaf(wr[k], xv[k], acc);
            if constexpr (decltype(has_bias)::value) acc = acc + bias[co];
            if constexpr (decltype(has_relu)::value) acc = relu_idiom(acc);
            trow[cc] = acc;
        }
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    const bool b = (flags & CAMEL_EPI_BIAS) != 0, r = (flags & CAMEL_EPI_RELU) != 0;
    for (int c0 = 0; c0 < Co; c0 += CH) {
        const int cw = min(CH, Co - c0); // a multiple of 4
        if (b && r)
            channels(T_{}, T_{}, c0, cw);
        else if (b)
            channels(T_{}, F_{}, c0, cw);
        else if (r)
            channels(F_{}, T_{}, c0, cw);
        else
            channels(F_{}, F_{}, c0, cw);
        __syncthreads();
        const int q4 = cw >> 2;
        for (int i = threadIdx.x; i < npix * q4; i += PIXB) {
            const int row = i / q4, q = i - row * q4;
            const float *t = tile + row * LD + 4 * q;
            *reinterpret_cast<float4 *>(y + (size_t)(pg0 + row) * Co + c0 + 4 * q) =
                make_float4(t[0], t[1], t[2], t[3]);
        }
        __syncthreads();
    }
}

// ---- host-side launch -----------------------------------------------------------

// Tile shapes, chosen by measured sweeps on MI355X (GEMM 1024-8192, the
// benchmark conv shapes 64x64x56x56 -> 128 and 512x32x26x26 -> 64, 3x3): 8
// waves at 256x256 keep the accumulators in arch
// VGPRs without spills; the conv tiles are small enough for two work-groups
// per CU, which hides the gather latency better than larger tiles do.
using TileBig = Tile<256, 256, 32, 2, 4, 1, false>; // wave 128x64, 8 waves
using TileMid = Tile<128, 128, 32, 2, 2>;           // wave 64x64
// One round of 128x128 tiles (at most one work-group per CU, e.g. 2048^3):
// 8 waves, two k-groups that take halves of each 64-k stage, loads two
// stages ahead (2048^3 121.4 -> 127.9 TFLOP/s; with two rounds the 4-wave
// tile stays ahead, 130.4 against 129.2 at 2048x4096x2048).
using TileMidK = Tile<128, 128, 64, 2, 2, 2, false>;
using TileSmall = Tile<64, 64, 64, 2, 2, 2>;        // wave 32x32, two k-groups (8 waves)
using TileTiny = Tile<32, 32, 64, 1, 1, 4>;         // one 32x32 block, four k-groups (4 waves)
using TileSkinny = Tile<32, 128, 64, 1, 4>;  // M <= 32 when the streaming kernel cannot run
using TileConv = Tile<128, 128, 32, 2, 2>;   // NHWC conv, Co > 64, C % 32 == 0
using TileConv16 = Tile<128, 128, 16, 2, 2>; // NHWC conv, Co > 64, C % 16 == 0
using TileConv64 = Tile<64, 128, 32, 2, 2>;  // NHWC conv, Co <= 64, C % 32 == 0
using TileConv64k16 = Tile<64, 128, 16, 2, 2>; // NHWC conv, Co <= 64, C % 16 == 0
using TileGather = Tile<128, 256, 16, 2, 2>;   // NCHW gather conv, Co > 64
using TileGather64 = Tile<64, 128, 32, 2, 2>;  // NCHW gather conv, Co <= 64 (no spills)

template <class T> int64_t tiles_of(int64_t M, int64_t N) {
    return ((M + T::BM - 1) / T::BM) * ((N + T::BN - 1) / T::BN);
}

// Scratch for split-K partials: a pool block grown on demand (kept for the
// process), or, while an allocation-free call runs, the library's static
// scratch (FixedPartials).  Callers hold the library lock throughout.
float *g_partial = nullptr;
size_t g_partial_bytes = 0;
float *g_fixed_partial = nullptr; // non-null only inside an allocation-free call
size_t g_fixed_partial_bytes = 0;

// Routes the partial sums of the calls made in its lifetime to a caller-
// provided buffer of `bytes` (the static scratch); nothing is allocated.
struct FixedPartials {
    FixedPartials(float *p, size_t bytes) {
        g_fixed_partial = p;
        g_fixed_partial_bytes = bytes;
    }
    ~FixedPartials() {
        g_fixed_partial = nullptr;
        g_fixed_partial_bytes = 0;
    }
    FixedPartials(const FixedPartials &) = delete;
    FixedPartials &operator=(const FixedPartials &) = delete;
};

// A buffer of at least `bytes` for split-K partials, into *out.
int partial_buffer(size_t bytes, float **out) {
    if (g_fixed_partial) {
        // The allocation-free entry points check their need up front.
        if (bytes > g_fixed_partial_bytes)
            return fail(CAMEL_HIP_ERR_SHAPE, "split-K partials exceed the static scratch");
        *out = g_fixed_partial;
        return CAMEL_HIP_OK;
    }
    if (bytes > g_partial_bytes) {
        if (g_partial) {
            CAMEL_RETURN_IF(check_hip(hipStreamSynchronize(stream()), "hipStreamSynchronize"));
            camel_hip_free(g_partial);
            g_partial = nullptr;
            g_partial_bytes = 0;
        }
        void *p = nullptr;
        CAMEL_RETURN_IF(camel_hip_malloc(&p, bytes));
        g_partial = static_cast<float *>(p);
        g_partial_bytes = bytes;
    }
    *out = g_partial;
    return CAMEL_HIP_OK;
}

// True when the streaming skinny kernel serves C[M, N] = A[M, K] B[K, N].
bool skinny_eligible(int64_t M, int64_t N, int64_t K, const float *B, const float *C) {
    return M <= 32 && K > 0 && N % 4 == 0 && ((uintptr_t)B & 15) == 0 &&
           ((uintptr_t)C & 15) == 0 && (K + SK_CHUNK - 1) / SK_CHUNK <= SK_MAX_KGROUPS;
}

// Shape of a skinny launch: chunks per work-group (ch) and work-groups along
// K (nks; their partials need nks * M * N floats when nks > 1).
struct SkinnyPlan {
    int ch, nks;
};

SkinnyPlan plan_skinny(int64_t N, int64_t K) {
    const int64_t strips = (N + SK_COLS - 1) / SK_COLS;
    // Chunks per work-group: the most that still leaves one work-group per
    // CU (fewer, longer streams measured faster than more, shorter ones).
    const int cus = std::max(1, device_cu_count());
    int ch = 1;
    for (int c : {8, 4, 2}) {
        if (strips * ((K + SK_CHUNK * c - 1) / (SK_CHUNK * c)) >= cus) {
            ch = c;
            break;
        }
    }
    return {ch, (int)((K + SK_CHUNK * ch - 1) / (SK_CHUNK * ch))};
}

size_t skinny_partial_bytes(int64_t M, int64_t N, int64_t K) {
    const SkinnyPlan p = plan_skinny(N, K);
    return p.nks > 1 ? (size_t)p.nks * M * N * sizeof(float) : 0;
}

int launch_skinny(const float *A, const float *B, float *C, int M, int N, int K, const float *bias,
                  int flags) {
    const int strips = (N + SK_COLS - 1) / SK_COLS;
    const int ch = plan_skinny(N, K).ch;
    const int mt = M <= 16 ? 1 : 2;
    const int a_vec = M >= 16 * mt && K % 4 == 0 && ((uintptr_t)A & 15) == 0;
    auto go = [&](auto kernel, int chunks) -> int {
        const int nks = (K + SK_CHUNK * chunks - 1) / (SK_CHUNK * chunks);
        float *partial = nullptr;
        if (nks > 1) CAMEL_RETURN_IF(partial_buffer((size_t)nks * M * N * sizeof(float), &partial));
        hipLaunchKernelGGL(kernel, dim3((unsigned)strips, (unsigned)nks), dim3(SK_WAVES * 64), 0,
                           stream(), A, B, C, M, N, K, bias, flags, partial, a_vec);
        CAMEL_RETURN_IF(check_launch("sgemm_skinny_kernel"));
        if (nks == 1) return CAMEL_HIP_OK;
        const int64_t total4 = (int64_t)M * N / 4;
        const int by_strip = N % SK_COLS == 0 ? strips : 0;
        const unsigned blocks =
            by_strip ? (unsigned)(by_strip * ((M + 3) / 4))
                     : (unsigned)((total4 + SK_REDUCE_THREADS - 1) / SK_REDUCE_THREADS);
        hipLaunchKernelGGL(skinny_reduce_kernel, dim3(blocks), dim3(SK_REDUCE_THREADS), 0, stream(),
                           reinterpret_cast<const float4 *>(partial), reinterpret_cast<float4 *>(C),
                           M, N, nks, bias, flags, by_strip);
        return check_launch("skinny_reduce_kernel");
    };
    if (mt == 1) {
        if (ch == 8) return go(sgemm_skinny_kernel<1, 8>, 8);
        if (ch == 4) return go(sgemm_skinny_kernel<1, 4>, 4);
        if (ch == 2) return go(sgemm_skinny_kernel<1, 2>, 2);
        return go(sgemm_skinny_kernel<1, 1>, 1);
    }
    if (ch == 8) return go(sgemm_skinny_kernel<2, 8>, 8);
    if (ch == 4) return go(sgemm_skinny_kernel<2, 4>, 4);
    if (ch == 2) return go(sgemm_skinny_kernel<2, 2>, 2);
    return go(sgemm_skinny_kernel<2, 1>, 1);
}

// Work-groups of one kernel that fit on the chip at once (occupancy x CUs).
template <class T, int AMODE, int BMODE> int resident_slots() {
    static int slots = 0;
    if (slots == 0) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, sgemm_kernel<T, AMODE, BMODE>,
                                                         T::THREADS, 0) != hipSuccess ||
            per_cu < 1)
            per_cu = 1;
        slots = per_cu * device_cu_count();
    }
    return slots;
}

// K range per split and the split count a launch really runs for a request
// of `splits`: whole BK stages per split, no empty split.
template <class T> void split_k(int K, int splits, int &k_per_split, int &used) {
    const int stages = (K + T::BK - 1) / T::BK;
    splits = std::max(1, std::min(splits, stages));
    const int kps_stages = (stages + splits - 1) / splits;
    k_per_split = std::max(1, kps_stages) * T::BK;
    used = std::max(1, (K + k_per_split - 1) / k_per_split);
}

// Partial-sum bytes of a launch of `ntiles` tiles asked to split K `splits`
// ways (0 when it runs unsplit and is not a partials-only launch).
template <class T> size_t range_partial_bytes(int K, int ntiles, int splits, bool partials_only) {
    int kps = 0, used = 1;
    split_k<T>(K, splits, kps, used);
    if (used <= 1 && !partials_only) return 0;
    return (size_t)used * ntiles * T::BM * T::BN * sizeof(float);
}

// Runs tiles [tile_begin, tile_begin + ntiles) with `splits` K splits; split
// launches write partials that tile_reduce_kernel folds into C.  With
// `partials_only` the reduce is left to the caller: *partials_only receives
// the split count and *partials_at the buffer the partials stay in.
template <class T, int AMODE, int BMODE>
int launch_range(GemmArgs g, int tile_begin, int ntiles, int splits, const char *name,
                 int *partials_only = nullptr, float **partials_at = nullptr) {
    g.tile_begin = tile_begin;
    split_k<T>(g.K, splits, g.k_per_split, splits);
    g.partial = nullptr;
    if (splits > 1 || partials_only) { // a partials-only launch writes partials even unsplit
        CAMEL_RETURN_IF(partial_buffer(
            (size_t)splits * ntiles * T::BM * T::BN * sizeof(float), &g.partial));
    }
    hipLaunchKernelGGL((sgemm_kernel<T, AMODE, BMODE>), dim3((unsigned)ntiles, (unsigned)splits),
                       dim3(T::THREADS), 0, stream(), g);
    CAMEL_RETURN_IF(check_launch(name));
    if (partials_only) {
        *partials_only = splits;
        if (partials_at) *partials_at = g.partial;
        return CAMEL_HIP_OK;
    }
    if (splits > 1) {
        const size_t total = (size_t)ntiles * T::BM * T::BN;
        if (is_pool<BMODE>)
            hipLaunchKernelGGL((tile_reduce_kernel<T::BM, T::BN, true, true>),
                               dim3(grid_for((int64_t)total / 4, 256)), dim3(256), 0, stream(), g,
                               ntiles, splits);
        else
            hipLaunchKernelGGL((tile_reduce_kernel<T::BM, T::BN, is_conv<BMODE>>),
                               dim3(grid_for((int64_t)total, 256)), dim3(256), 0, stream(), g,
                               ntiles, splits);
        CAMEL_RETURN_IF(check_launch("tile_reduce_kernel"));
    }
    return CAMEL_HIP_OK;
}

// Small tile for the column band left after the whole rounds (see run_gemm):
// 64 x 32 with 4 waves (2 x 1 spatial x 2 k-groups, so all 4 SIMDs of a CU
// work on it); 64 x 64 with 2 x 2 waves when BK = 16, which two k-groups
// would not split into whole 8-k groups per register buffer.
template <class T>
using BandTile = Tile<64, (T::BK >= 32 ? 32 : 64), T::BK, 2, (T::BK >= 32 ? 1 : 2),
                      (T::BK >= 32 ? 2 : 1)>;
using BandTile64 = Tile<64, 32, 64, 2, 1, 2>;

// Schedules all tiles.  `splits` > 1 splits every tile (small problems).
// Otherwise whole rounds of resident work-groups run as whole tiles, and the
// tiles of a last, partial round (when it is at most a quarter full) run so
// that the whole chip shares them instead of leaving most CUs idle for a
// whole tile time:
//   * when every tile row sits in one tile-row group (tile id = tn * tiles_m
//     + tm) the leftover tiles are whole tile columns, i.e. a column band,
//     and that band runs as one launch of small tiles over all of K (no
//     partials; measured faster than the split below at the 64x64x56x56
//     -> 128 3x3 conv,
//     whose 1568 tiles leave 32 after 3 rounds);
//   * otherwise the leftover tiles are split along K and reduced in order.
// The launches run_gemm makes: tiles [0, head) unsplit (or all tiles with
// `head_splits` when the caller split every tile), then either nothing, a
// column band of small tiles from column band_n, or tiles [head, head + tail)
// with tail_splits K splits.
struct GemmSchedule {
    int head = 0, head_splits = 1;
    bool band = false;
    int band_n = 0;
    int tail = 0, tail_splits = 1;
};

template <class T, int AMODE, int BMODE> GemmSchedule schedule_gemm(const GemmArgs &g, int splits) {
    GemmSchedule s;
    const int tiles_m = (g.M + T::BM - 1) / T::BM;
    const int tiles = (int)((int64_t)tiles_m * ((g.N + T::BN - 1) / T::BN));
    s.head = tiles;
    if (splits > 1) {
        s.head_splits = splits;
        return s;
    }
    const int slots = resident_slots<T, AMODE, BMODE>();
    const int stages = (g.K + T::BK - 1) / T::BK;
    const int full = tiles / slots, rem = tiles % slots;
    if (full == 0 || rem == 0 || stages < 4 || rem * 4 > slots) return s;
    s.head = full * slots;
    if (tiles_m <= GROUP_M && rem % tiles_m == 0) {
        s.band = true;
        s.band_n = s.head / tiles_m * T::BN;
        return s;
    }
    s.tail = rem;
    s.tail_splits = std::max(1, std::min(slots / rem, stages / 2));
    return s;
}

// Partial-sum bytes the schedule needs (the band runs unsplit).
template <class T> size_t schedule_partial_bytes(const GemmArgs &g, const GemmSchedule &s) {
    return std::max(range_partial_bytes<T>(g.K, s.head, s.head_splits, false),
                    s.tail ? range_partial_bytes<T>(g.K, s.tail, s.tail_splits, false) : 0);
}

template <class T, int AMODE, int BMODE> int run_gemm(GemmArgs g, int splits, const char *name) {
    const GemmSchedule s = schedule_gemm<T, AMODE, BMODE>(g, splits);
    CAMEL_RETURN_IF((launch_range<T, AMODE, BMODE>(g, 0, s.head, s.head_splits, name)));
    if (s.band) {
        GemmArgs band = g;
        band.n_begin = s.band_n;
        if constexpr (T::BK == 32 && is_nhwc<BMODE>) {
            // stages of 64 channels where the channels allow (a stage stays
            // within one (kh, kw)): half the stages of the latency-bound
            // small tiles (config-4 conv: 268.9 -> 266.2 us per call)
            if (g.Cin % 64 == 0) {
                using TB = BandTile64;
                const int band_tiles = (int)((int64_t)((g.M + TB::BM - 1) / TB::BM) *
                                             ((g.N - band.n_begin + TB::BN - 1) / TB::BN));
                return launch_range<TB, AMODE, BMODE>(band, 0, band_tiles, 1, name);
            }
        }
        using TB = BandTile<T>;
        const int band_tiles =
            (int)((int64_t)((g.M + TB::BM - 1) / TB::BM) * ((g.N - band.n_begin + TB::BN - 1) / TB::BN));
        // the band's small tiles take the register loaders (LOAD_DMA is for
        // 64-column tiles)
        constexpr int BA = AMODE == LOAD_DMA ? LOAD_VEC : AMODE;
        constexpr int BB = BMODE == LOAD_DMA ? LOAD_VEC : BMODE;
        return launch_range<TB, BA, BB>(band, 0, band_tiles, 1, name);
    }
    if (s.tail) return launch_range<T, AMODE, BMODE>(g, s.head, s.tail, s.tail_splits, name);
    return CAMEL_HIP_OK;
}

// True when the LOAD_DMA stage loop can run g: a tile shape it serves,
// row-major operands with 16-byte rows (avec, bvec, 16-byte aligned leading
// dimensions) and every tile inside M x N (the DMAs have no guards; only a
// ragged first K stage is loaded with them).
template <class T> bool dma_eligible(const GemmArgs &g, bool avec, bool bvec) {
    if constexpr (dma_tile<T>)
        return avec && bvec && g.M % T::BM == 0 && (g.N - g.n_begin) % T::BN == 0 &&
               g.lda % 4 == 0 && g.ldb % 4 == 0;
    return false;
}

// Runs the tile GEMM with the loaders the operands allow: A row-major or
// (atrans) given transposed, each with 16-byte loads where avec / bvec.
template <class T> int launch_gemm_modes(GemmArgs g, int splits, bool avec, bool bvec,
                                         bool atrans = false) {
    if constexpr (dma_tile<T>) {
        if (!atrans && dma_eligible<T>(g, avec, bvec))
            return run_gemm<T, LOAD_DMA, LOAD_DMA>(g, splits, "sgemm_kernel");
    }
    if (atrans) {
        if (avec && bvec) return run_gemm<T, LOAD_TVEC, LOAD_VEC>(g, splits, "sgemm_kernel");
        if (avec) return run_gemm<T, LOAD_TVEC, LOAD_SCALAR>(g, splits, "sgemm_kernel");
        if (bvec) return run_gemm<T, LOAD_TSCALAR, LOAD_VEC>(g, splits, "sgemm_kernel");
        return run_gemm<T, LOAD_TSCALAR, LOAD_SCALAR>(g, splits, "sgemm_kernel");
    }
    if (avec && bvec) return run_gemm<T, LOAD_VEC, LOAD_VEC>(g, splits, "sgemm_kernel");
    if (avec) return run_gemm<T, LOAD_VEC, LOAD_SCALAR>(g, splits, "sgemm_kernel");
    if (bvec) return run_gemm<T, LOAD_SCALAR, LOAD_VEC>(g, splits, "sgemm_kernel");
    return run_gemm<T, LOAD_SCALAR, LOAD_SCALAR>(g, splits, "sgemm_kernel");
}

// Partial-sum bytes launch_gemm_modes<T> will need for these arguments.
template <class T> size_t gemm_modes_partial_bytes(const GemmArgs &g, int splits, bool avec,
                                                   bool bvec, bool atrans = false) {
    GemmSchedule s;
    bool dma = false;
    if constexpr (dma_tile<T>) dma = !atrans && dma_eligible<T>(g, avec, bvec);
    if (dma) {
        if constexpr (dma_tile<T>) s = schedule_gemm<T, LOAD_DMA, LOAD_DMA>(g, splits);
    } else if (atrans) {
        if (avec && bvec)
            s = schedule_gemm<T, LOAD_TVEC, LOAD_VEC>(g, splits);
        else if (avec)
            s = schedule_gemm<T, LOAD_TVEC, LOAD_SCALAR>(g, splits);
        else if (bvec)
            s = schedule_gemm<T, LOAD_TSCALAR, LOAD_VEC>(g, splits);
        else
            s = schedule_gemm<T, LOAD_TSCALAR, LOAD_SCALAR>(g, splits);
    } else if (avec && bvec)
        s = schedule_gemm<T, LOAD_VEC, LOAD_VEC>(g, splits);
    else if (avec)
        s = schedule_gemm<T, LOAD_VEC, LOAD_SCALAR>(g, splits);
    else if (bvec)
        s = schedule_gemm<T, LOAD_SCALAR, LOAD_VEC>(g, splits);
    else
        s = schedule_gemm<T, LOAD_SCALAR, LOAD_SCALAR>(g, splits);
    return schedule_partial_bytes<T>(g, s);
}

// The split-K launch run_gemm makes for `splits` > 1, without its reduce:
// the partials of all tiles stay in g_partial for a consumer that finishes
// them (SplitPartialsA).  Fills the geometry that consumer needs.
template <class T>
int launch_split_partials(GemmArgs g, int splits, bool avec, bool bvec, SplitPartialsA &out) {
    const int tiles_m = (g.M + T::BM - 1) / T::BM, tiles_n = (g.N + T::BN - 1) / T::BN;
    const int tiles = tiles_m * tiles_n;
    int used = 0;
    float *at = nullptr;
    bool dma = false;
    if constexpr (dma_tile<T>) dma = dma_eligible<T>(g, avec, bvec);
    if (dma) {
        if constexpr (dma_tile<T>)
            CAMEL_RETURN_IF((launch_range<T, LOAD_DMA, LOAD_DMA>(g, 0, tiles, splits, "sgemm_kernel", &used, &at)));
    } else if (avec && bvec)
        CAMEL_RETURN_IF((launch_range<T, LOAD_VEC, LOAD_VEC>(g, 0, tiles, splits, "sgemm_kernel", &used, &at)));
    else if (avec)
        CAMEL_RETURN_IF((launch_range<T, LOAD_VEC, LOAD_SCALAR>(g, 0, tiles, splits, "sgemm_kernel", &used, &at)));
    else if (bvec)
        CAMEL_RETURN_IF((launch_range<T, LOAD_SCALAR, LOAD_VEC>(g, 0, tiles, splits, "sgemm_kernel", &used, &at)));
    else
        CAMEL_RETURN_IF((launch_range<T, LOAD_SCALAR, LOAD_SCALAR>(g, 0, tiles, splits, "sgemm_kernel", &used, &at)));
    out.partial = at;
    out.bias = g.bias;
    out.flags = g.flags;
    out.splits = used;
    out.ntiles = tiles;
    out.tiles_m = tiles_m;
    out.tiles_n = tiles_n;
    out.BM = T::BM;
    out.BN = T::BN;
    return CAMEL_HIP_OK;
}

enum class Cfg { Big, Mid, MidK, Small, Tiny, Skinny };

// Picks a tile shape and split count so the grid covers the chip's CUs.
void choose(int64_t M, int64_t N, int64_t K, int cus, Cfg &cfg, int &splits, int &bk) {
    splits = 1;
    int64_t tiles;
    if (M <= 32) {
        cfg = Cfg::Skinny;
        bk = TileSkinny::BK;
        tiles = tiles_of<TileSkinny>(M, N);
    } else if (tiles_of<TileBig>(M, N) >= cus) {
        cfg = Cfg::Big;
        bk = TileBig::BK;
        return;
    } else if (tiles_of<TileMid>(M, N) >= cus) {
        cfg = Cfg::Mid;
        bk = TileMid::BK;
        return;
    } else {
        cfg = Cfg::Small;
        bk = TileSmall::BK;
        tiles = tiles_of<TileSmall>(M, N);
        if (tiles >= cus) return;
    }
    // Split K so tiles*splits fills the chip, keeping >= 4 stages per split.
    auto split_for = [&](int64_t t) {
        const int64_t want = (cus + t - 1) / t;
        const int64_t max_splits = std::max<int64_t>(1, K / (4 * bk));
        return (int)std::max<int64_t>(1, std::min<int64_t>(want, std::min<int64_t>(max_splits, 64)));
    };
    splits = split_for(tiles);
    // A short K leaves too few 64 x 64 work-groups to cover half the CUs
    // (e.g. the 256^3 matmul: 16): 32 x 32 tiles, four times as many
    // (256^3: 7.5 -> 5.0 us).  Not when splits already fill the chip (the
    // CNN's 512x9216 -> 128 layer measured 21 us with 64 x 64 x 16 splits
    // against 30 us with 32 x 32 x 4).
    if (cfg == Cfg::Small && tiles * splits * 2 < cus) {
        cfg = Cfg::Tiny;
        tiles = tiles_of<TileTiny>(M, N);
        splits = split_for(tiles);
    }
}

// ---- the first two convolutions of an image CNN, fused with the pool -----------
//
// y = maxpool2x2(conv2(conv1(x))) (each conv with its optional bias and relu)
// for a one-channel input: conv1 1 -> CP_C1 channels, 3x3, then conv2
// CP_C1 -> Co2, 3x3, both stride 1 and unpadded, then the 2x2 stride-2 pool.
// conv1's output (CP_C1 x 26 x 26 per 28 x 28 image, 44 MB at batch 512)
// never reaches HBM: a work-group computes the rows of it that its band of
// conv2 rows reads into LDS, then runs conv2 as an implicit GEMM whose B
// operand is read straight from that LDS patch, and stores only the pooled
// values.
//   * work-group = (image, band of CP_BR pooled rows = 2 CP_BR conv2 rows) x
//     64 output channels; 4 waves as 2 (channels) x 2 (column halves), each
//     wave 32 channels x CP_NBW blocks of 32 columns;
//   * columns in pool order, 4 per window ((0,0), (0,1), (1,0), (1,1)), so a
//     window is one DPP quad and the epilogue takes its max in registers,
//     and 16 consecutive columns a 2 x 2 block of windows (cp_window);
//   * conv1 is the direct kernel's FMA chain (k = (kh, kw) ascending, then
//     bias and x * (x > 0)), so the patch holds exactly the values the conv1
//     kernel stores;
//   * conv2's A operand (weights packed [Co2][3][3][CP_C1]) is held in
//     registers for all of K; the MFMA sequence -- K in (kh, kw, c) order,
//     8-channel groups, each 32x32x2 MFMA pairing channels c and c + 4 --
//     and the epilogue (bias, relu, strict-'>' window max) are those of the
//     implicit GEMM with the pooled NCHW4 loader, so the result equals the
//     two conv calls and the pool bit for bit.
constexpr int CP_C1 = 32;                 // conv1 output channels = conv2 input channels
constexpr int CP_W = 28;                  // input width
constexpr int CP_OW1 = CP_W - 2;          // conv1 output width (26)
constexpr int CP_PW = (CP_OW1 - 2) / 2;   // pooled width (12)
constexpr int CP_BR = 4;                  // pooled rows per work-group
constexpr int CP_R1 = 2 * CP_BR + 2;      // conv1 rows a band reads (10)
constexpr int CP_IR = CP_R1 + 2;          // input rows a band reads (12)
// The patch is stored by channel quads, [C1/4][CP_R1][CP_RS][4]: a lane reads
// the 4 channels of one pixel that 4 consecutive MFMAs take with one 16-byte
// read.  A 16-byte LDS read serves 16 lanes per clock, conflict-free when
// their chunks are distinct mod 16 (64 banks x 4 bytes); those 16 lanes read
// a 2 x 2 block of windows, pixels (2 py + r, 2 px + c) for r, c in 0..3, and
// with a row pitch of CP_RS = 28 pixels (28 r = 0, 12, 8, 4 mod 16) the 16
// chunks are distinct.  (4 windows of one row, 2 rows x 8 pixels, put 4
// chunks on 2 lanes each at this pitch; a pitch of 40 separates those too but
// ran the CNN forward 1.7% slower; the 2 x 2 blocks ran it 0.4% faster.  The
// kernel's SQ_LDS_BANK_CONFLICT share reads 28.5% with either mapping at this
// pitch and 0 at pitch 40, so what that counter counts here is not explained
// by this model of the patch reads.)
constexpr int CP_RS = 28;
static_assert(CP_RS >= CP_OW1 && CP_RS % 16 == 12, "conflict-free patch row pitch");
// One channel quad of the patch: 1120 floats, padded to 1124 (= 4 mod 32) so
// that the conv1 phase's 32 lanes, one channel each, store one pixel to 32
// distinct banks.
constexpr int CP_QPLANE = CP_R1 * CP_RS * 4 + 4;
constexpr int CP_COLS = CP_BR * CP_PW * 4; // GEMM columns of a band (192)
constexpr int CP_NBW = CP_COLS / 32 / 2;  // 32-column blocks per wave (3)
static_assert(CP_COLS % 64 == 0, "a band is whole 32-column blocks for both column halves");

// The pool window (row py of the band, column px) of GEMM column col: 4
// columns per window, and 16 consecutive columns a 2 x 2 block of windows.
__device__ __forceinline__ void cp_window(int col, int &py, int &px) {
    static_assert(CP_BR % 2 == 0 && CP_PW % 2 == 0, "windows in 2 x 2 blocks");
    const int g = col >> 4, w4 = (col >> 2) & 3;
    py = 2 * (g / (CP_PW / 2)) + (w4 >> 1);
    px = 2 * (g % (CP_PW / 2)) + (w4 & 1);
}

__global__ __launch_bounds__(256, 2) void conv_pair_pool_kernel(
    const float *__restrict__ x, const float *__restrict__ w1, const float *__restrict__ b1,
    const float *__restrict__ w2p, const float *__restrict__ b2, float *__restrict__ y, int H,
    int Co2, int bands, int flags1, int flags2) {
    const bool BIAS1 = flags1 & CAMEL_EPI_BIAS, RELU1 = flags1 & CAMEL_EPI_RELU;
    const bool BIAS2 = flags2 & CAMEL_EPI_BIAS, RELU2 = flags2 & CAMEL_EPI_RELU;
    __shared__ __attribute__((aligned(16))) float patch[CP_C1 / 4 * CP_QPLANE];
    __shared__ __attribute__((aligned(16))) float img[CP_IR * CP_W];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int half = lane >> 5, r32 = lane & 31;
    const int wm = wave & 1, wn = wave >> 1;
    const int n = blockIdx.x / bands, band = blockIdx.x - n * bands;
    const int m0 = blockIdx.y * 64;
    const int PH = bands * CP_BR;
    const int Y0 = band * 2 * CP_BR; // first conv2 (and conv1) row of the band

    // conv2 weights of this lane's row as the MFMA A operand, one (kh, kw)
    // at a time: a[buf][s8] holds channels 8 s8 + 4 half .. +3 (from L2,
    // two (kh, kw) ahead of their use).
    const float *wr = w2p + (size_t)(m0 + 32 * wm + r32) * 9 * CP_C1 + 4 * half;
    float4 a[3][CP_C1 / 8];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int s8 = 0; s8 < CP_C1 / 8; ++s8)
            a[j][s8] = *reinterpret_cast<const float4 *>(wr + j * CP_C1 + 8 * s8);

    // conv1's weights and bias for this lane's channel (lane r32 computes
    // channel r32 of one pixel; the two half-waves take two pixels).
    float w1r[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) w1r[k] = w1[r32 * 9 + k];
    const float b1r = BIAS1 ? b1[r32] : 0.f;

    // The input rows of the band, 16 bytes per thread (zeros past the image:
    // never read by a valid output, since the bands tile the pooled rows).
    {
        const float4 *xi = reinterpret_cast<const float4 *>(x + ((size_t)n * H + Y0) * CP_W);
        if (tid < CP_IR * CP_W / 4) {
            const int r = Y0 + tid / (CP_W / 4);
            reinterpret_cast<float4 *>(img)[tid] = r < H ? xi[tid] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    __syncthreads();

    // conv1 into the patch: the direct kernel's FMA chain, then bias and relu.
    for (int p = 2 * wave + half; p < CP_R1 * CP_OW1; p += 8) {
        const int r = p / CP_OW1, c = p - r * CP_OW1;
        float acc = 0.f;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
            for (int kw = 0; kw < 3; ++kw)
                acc = __builtin_fmaf(w1r[kh * 3 + kw], img[(r + kh) * CP_W + c + kw], acc);
        if (BIAS1) acc = acc + b1r;
        if (RELU1) acc = relu_idiom(acc);
        patch[(r32 >> 2) * CP_QPLANE + (r * CP_RS + c) * 4 + (r32 & 3)] = acc;
    }
    __syncthreads();

    // conv2: lane (r32, half) reads B[k][col] for channels 8 s8 + 4 half + t,
    // t = 0..3, of pixel (oy + kh, ox + kw) of its column col of each block:
    // one 16-byte read of channel quad 2 s8 + half.
    int base[CP_NBW];
#pragma unroll
    for (int b = 0; b < CP_NBW; ++b) {
        const int col = 32 * (CP_NBW * wn + b) + r32, d = col & 3;
        int py, px;
        cp_window(col, py, px);
        base[b] = half * CP_QPLANE + ((2 * py + (d >> 1)) * CP_RS + 2 * px + (d & 1)) * 4;
    }
    floatx16 acc[CP_NBW];
#pragma unroll
    for (int b = 0; b < CP_NBW; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][v] = 0.f;
    // Each 8-channel group of a (kh, kw) stage loads the same group's weights
    // of stage + 2 and reads the next group's patch values, spread over its
    // own MFMAs: one patch read per two MFMAs, then the weight load
    // (scheduling group barriers keep that order; 4% faster over the CNN
    // forward than the reads together ahead of the MFMAs and the stage's
    // weight loads together at its start).
    auto patch_reads = [&](int khw, int s8, float4 *bv) {
        const int kh = khw / 3, kw = khw - 3 * (khw / 3);
        const int off = 2 * s8 * CP_QPLANE + (kh * CP_RS + kw) * 4;
#pragma unroll
        for (int b = 0; b < CP_NBW; ++b)
            bv[b] = *reinterpret_cast<const float4 *>(patch + base[b] + off);
    };
    float4 bv[2][CP_NBW];
    patch_reads(0, 0, bv[0]);
#pragma unroll
    for (int khw = 0; khw < 9; ++khw) {
        const int cur = khw % 3;
#pragma unroll
        for (int s8 = 0; s8 < CP_C1 / 8; ++s8) {
            const int g = khw * (CP_C1 / 8) + s8; // group index over all of K
            const bool next = g + 1 < 9 * (CP_C1 / 8);
            const bool ahead = khw + 2 < 9;
            // group s8's weights of stage khw + 2
            if (ahead)
                a[(khw + 2) % 3][s8] =
                    *reinterpret_cast<const float4 *>(wr + (khw + 2) * CP_C1 + 8 * s8);
            if (next) patch_reads((g + 1) / (CP_C1 / 8), (g + 1) % (CP_C1 / 8), bv[(g + 1) & 1]);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int b = 0; b < CP_NBW; ++b)
                    acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[cur][s8][t], bv[g & 1][b][t],
                                                                  acc[b], 0, 0, 0);
            if (next) {
                // one patch read per two MFMAs at the head of the group, then
                // the weight load after one more MFMA (masks: 0x100 LDS read,
                // 0x20 global read, 0x8 MFMA)
#pragma unroll
                for (int r = 0; r < CP_NBW; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                if (ahead) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 2 * CP_NBW - 1, 0);
                } else {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2 * CP_NBW, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Epilogue: bias, relu, then the window max over the lane quad in the
    // order (0,0), (0,1), (1,0), (1,1) with a strict '>'; the quad's first
    // lane stores the pooled value.
    float brow[16];
#pragma unroll
    for (int v = 0; v < 16; ++v)
        brow[v] = BIAS2 ? b2[m0 + 32 * wm + 8 * (v >> 2) + 4 * half + (v & 3)] : 0.f;
#pragma unroll
    for (int b = 0; b < CP_NBW; ++b) {
        const int col = 32 * (CP_NBW * wn + b) + r32;
        int py, px;
        cp_window(col, py, px);
        py += band * CP_BR;
        float *out = y + ((size_t)n * Co2 + m0 + 32 * wm) * PH * CP_PW + (size_t)py * CP_PW + px;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = 8 * (v >> 2) + 4 * half + (v & 3);
            float xo = acc[b][v];
            if (BIAS2) xo = xo + brow[v];
            if (RELU2) xo = relu_idiom(xo);
            const float x1 = quad_lane<1>(xo), x2 = quad_lane<2>(xo), x3 = quad_lane<3>(xo);
            float mx = xo;
            if (x1 > mx) mx = x1;
            if (x2 > mx) mx = x2;
            if (x3 > mx) mx = x3;
            if ((r32 & 3) == 0) out[(size_t)row * PH * CP_PW] = mx;
        }
    }
}

// True when conv_pair_pool_kernel serves the pair.
bool conv_pair_supported(int64_t H, int64_t W, int64_t C1, int64_t Co2) {
    return W == CP_W && C1 == CP_C1 && Co2 > 0 && Co2 % 64 == 0 && H >= 6 &&
           (H - 4) % (2 * CP_BR) == 0;
}

// ---- conv2d host paths -----------------------------------------------------------

// Activation layouts of the conv paths: NCHW (the tensor layout), NHWC and
// NCHW4 ([N][C/4][H][W][4]), the last two chosen by the layout flags.
enum Layout { L_NCHW, L_NHWC, L_NCHW4 };

int conv2d_direct(const float *x, const float *w, const float *bias, float *y, int64_t N, int64_t C,
                  int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW, int64_t stride,
                  int64_t pad, int64_t OH, int64_t OW, int flags, Layout y_layout) {
    const int64_t P = OH * OW, NP = N * P;
    const int64_t K = C * KH * KW;
    if (y_layout == L_NHWC) {
        // Co % 4 == 0 and y 16-byte aligned (checked by the caller)
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3((unsigned)((NP + DN_PIX - 1) / DN_PIX)), dim3(DN_PIX), 0, stream(),
                               x, w, bias, y, (int)NP, (int)P, (int)OW, (int)C, (int)H, (int)W,
                               (int)Co, (int)KH, (int)KW, (int)stride, (int)pad, flags);
            return check_launch("conv2d_direct_nhwc_kernel");
        };
        if (K == 9) return go(conv2d_direct_nhwc_kernel<9, true>);
        if (K == 25) return go(conv2d_direct_nhwc_kernel<25, true>);
        if (K == 27) return go(conv2d_direct_nhwc_kernel<27, true>);
        if (K <= 16) return go(conv2d_direct_nhwc_kernel<16, false>);
        return go(conv2d_direct_nhwc_kernel<DIRECT_MAX_K, false>);
    }
    // 2 pixels per thread (8-byte stores) when every channel plane of y
    // stays 8-byte aligned (measured 2-4% faster than 1 or 4 at the CNN's
    // first layer); 1 otherwise.
    const bool pair = P % 2 == 0 && ((uintptr_t)y & 7) == 0;
    auto go = [&](auto kernel, int pix) {
        const int64_t threads = (NP + pix - 1) / pix;
        hipLaunchKernelGGL(kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream(), x,
                           w, bias, y, (int)NP, (int)P, (int)OW, (int)C, (int)H, (int)W, (int)Co,
                           (int)KH, (int)KW, (int)stride, (int)pad, flags);
        return check_launch("conv2d_direct_kernel");
    };
    if (y_layout == L_NCHW4) {
        // Co % 4 == 0 and y 16-byte aligned (checked by the caller).  One
        // pixel per thread: each 16-byte store instruction then writes one
        // contiguous 1 KiB run of a channel-quad plane (two pixels per
        // thread interleave two instructions over 2 KiB: 13.0 against
        // 11.4 us at the CNN's first layer; four: 14.7 us).
        if (K == 9) return go(conv2d_direct_kernel<9, true, 1, true>, 1);
        if (K == 25) return go(conv2d_direct_kernel<25, true, 1, true>, 1);
        if (K == 27) return go(conv2d_direct_kernel<27, true, 1, true>, 1);
        if (K <= 16) return go(conv2d_direct_kernel<16, false, 1, true>, 1);
        return go(conv2d_direct_kernel<DIRECT_MAX_K, false, 1, true>, 1);
    }
    // Exact kernels for the usual first layers: 3x3 and 5x5 over 1 or 3
    // channels.
    if (K == 9)
        CAMEL_RETURN_IF(pair ? go(conv2d_direct_kernel<9, true, 2>, 2)
                             : go(conv2d_direct_kernel<9, true, 1>, 1));
    else if (K == 25)
        CAMEL_RETURN_IF(pair ? go(conv2d_direct_kernel<25, true, 2>, 2)
                             : go(conv2d_direct_kernel<25, true, 1>, 1));
    else if (K == 27)
        CAMEL_RETURN_IF(pair ? go(conv2d_direct_kernel<27, true, 2>, 2)
                             : go(conv2d_direct_kernel<27, true, 1>, 1));
    else if (K <= 16)
        CAMEL_RETURN_IF(go(conv2d_direct_kernel<16, false, 1>, 1));
    else
        CAMEL_RETURN_IF(go(conv2d_direct_kernel<DIRECT_MAX_K, false, 1>, 1));
    return ok();
}

// dst[n] = transpose of src[n] for n < N, each image an [A][B] matrix (NCHW
// -> NHWC with A = channels, B = pixels; NHWC -> NCHW with A = pixels, B =
// channels).  The transpose kernel's weight slice is given no weights.
int transpose_images(const float *src, float *dst, int64_t N, int64_t A, int64_t B) {
    if (N + 1 > 65535) return fail(CAMEL_HIP_ERR_SHAPE, "conv2d: batch too large for an NHWC layout");
    const bool vec = A % 4 == 0 && B % 4 == 0 && (((uintptr_t)src | (uintptr_t)dst) & 15) == 0;
    const int tp = vec ? TP_VEC : 32;
    dim3 grid((unsigned)((B + tp - 1) / tp), (unsigned)((A + 31) / 32), (unsigned)(N + 1));
    if (vec)
        hipLaunchKernelGGL(nchw_to_nhwc_kernel<true>, grid, dim3(256), 0, stream(), src, dst, (int)A,
                           (int)B, nullptr, nullptr, 0, 1);
    else
        hipLaunchKernelGGL(nchw_to_nhwc_kernel<false>, grid, dim3(256), 0, stream(), src, dst,
                           (int)A, (int)B, nullptr, nullptr, 0, 1);
    return check_launch("nchw_to_nhwc_kernel");
}

// NCHW -> NCHW4 (to_q4) or back, for `quads` = N*C/4 channel quads of HW
// pixels; the NCHW4 side 16-byte aligned.
int quad_layout(const float *src, float *dst, int64_t quads, int64_t HW, bool to_q4) {
    if (quads * HW == 0) return ok();
    const dim3 grid(grid_for(quads * HW, 256));
    if (to_q4)
        hipLaunchKernelGGL(quad_layout_kernel<true>, grid, dim3(256), 0, stream(), src, dst, quads,
                           (int)HW);
    else
        hipLaunchKernelGGL(quad_layout_kernel<false>, grid, dim3(256), 0, stream(), src, dst, quads,
                           (int)HW);
    return check_launch("quad_layout_kernel");
}

// w [Co][C][KHW] -> wp [Co][KHW][C] (the K order (kh, kw, c) of the NHWC
// implicit GEMM): the transpose kernel's weight slice, launched alone (a
// grid of one z slice is all weight slice).  With C and KHW exchanged the
// same launch unpacks.
int pack_weights(const float *w, float *wp, int64_t Co, int64_t C, int64_t KHW) {
    hipLaunchKernelGGL(nchw_to_nhwc_kernel<false>, dim3(grid_for(Co * C * KHW, 256), 1, 1),
                       dim3(256), 0, stream(), nullptr, nullptr, (int)C, 0, w, wp, (int)Co,
                       (int)KHW);
    return check_launch("nchw_to_nhwc_kernel");
}

// Pooled scratch owned for the duration of one entry point call (returned
// to the stream-ordered pool on scope exit).
struct Scratch {
    void *p = nullptr;
    ~Scratch() {
        if (p) camel_hip_free(p);
    }
    int alloc(size_t bytes) { return camel_hip_malloc(&p, bytes); }
    float *f() const { return static_cast<float *>(p); }
};

GemmArgs conv_args(const float *w, const float *x, const float *bias, float *y, int64_t N,
                   int64_t C, int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW,
                   int64_t stride, int64_t pad, int64_t OH, int64_t OW, int flags) {
    GemmArgs g{};
    g.A = w;
    g.B = x;
    g.C = y;
    g.bias = bias;
    g.M = (int)Co;
    g.N = (int)(N * OH * OW);
    g.K = (int)(C * KH * KW);
    g.lda = g.K;
    g.flags = flags;
    g.P = (int)(OH * OW);
    g.OW = (int)OW;
    g.H = (int)H;
    g.W = (int)W;
    g.CHW = (int)(C * H * W);
    g.stride = (int)stride;
    g.pad = (int)pad;
    g.Cin = (int)C;
    g.KW = (int)KW;
    g.pxs = (int)C; // NHWC
    g.cqs = 4;
    return g;
}

// Implicit GEMM over K ordered (kh, kw, c), x read in place: NHWC and NCHW4
// with one 16-byte load per k-quad of a pixel, NCHW with one load per channel
// plane (LOAD_PLANES; against transposing x to NHWC first, which moved 2 x
// 51 MB more per call: config-4 conv 291 -> 287 us, the CNN's conv2 from
// NCHW 160 -> 154 us).  w is reordered to (kh, kw, c) in pooled scratch
// (stream-ordered, returned to the pool after the launch) unless it comes
// packed.  pool: y is the 2x2 stride-2 max pool of the convolution,
// [N][Co][OH/2][OW/2], written from the GEMM epilogue.
template <class T>
int conv2d_nhwc(const float *x, const float *w, const float *bias, float *y, int64_t N, int64_t C,
                int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW, int64_t stride,
                int64_t pad, int64_t OH, int64_t OW, int flags, Layout x_layout, bool pool,
                bool w_packed) {
    const bool planes = x_layout == L_NCHW;
    const int64_t HW = H * W, K = C * KH * KW;
    Scratch wt;
    if (!w_packed) {
        CAMEL_RETURN_IF(wt.alloc((size_t)(Co * K) * sizeof(float)));
        CAMEL_RETURN_IF(pack_weights(w, wt.f(), Co, C, KH * KW));
    }
    GemmArgs g = conv_args(w_packed ? w : wt.f(), x, bias, y, N, C, H, W, Co, KH, KW, stride, pad,
                           OH, OW, flags);
    if (x_layout == L_NCHW4) {
        g.pxs = 4;
        g.cqs = (int)(4 * HW);
    } else if (planes) {
        g.pxs = 1;
        g.cqs = (int)(4 * HW);
        g.chs = (int)HW;
    }
    if (pool) {
        g.PW = (int)(OW / 2);
        g.PP = (int)((OH / 2) * (OW / 2));
        g.N = (int)(N * g.PP * 4);
        if (planes)
            CAMEL_RETURN_IF((run_gemm<T, LOAD_VEC, LOAD_PLANES_POOL>(g, 1, "conv2d_pool_kernel")));
        else
            CAMEL_RETURN_IF((run_gemm<T, LOAD_VEC, LOAD_NHWC_POOL>(g, 1, "conv2d_pool_kernel")));
    } else if (planes) {
        CAMEL_RETURN_IF((run_gemm<T, LOAD_VEC, LOAD_PLANES>(g, 1, "conv2d_planes_kernel")));
    } else {
        CAMEL_RETURN_IF((run_gemm<T, LOAD_VEC, LOAD_NHWC>(g, 1, "conv2d_nhwc_kernel")));
    }
    return ok();
}

// General path: im2col columns gathered from NCHW x through a k -> (c, kh, kw)
// offset table built on the host once per geometry.
int conv2d_gather(const float *x, const float *w, const float *bias, float *y, int64_t N,
                  int64_t C, int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW,
                  int64_t stride, int64_t pad, int64_t OH, int64_t OW, int flags) {
    const int64_t K = C * KH * KW;
    static std::vector<int2> host_tab;
    static int2 *dev_tab = nullptr;
    static int64_t tab_cap = 0;
    static int64_t tab_key[4] = {-1, -1, -1, -1};
    if (tab_key[0] != C || tab_key[1] != KH || tab_key[2] != KW || tab_key[3] != H * W * 65536 + W) {
        if (K > tab_cap) {
            if (dev_tab) {
                CAMEL_RETURN_IF(check_hip(hipStreamSynchronize(stream()), "hipStreamSynchronize"));
                camel_hip_free(dev_tab);
            }
            void *p = nullptr;
            CAMEL_RETURN_IF(camel_hip_malloc(&p, (size_t)K * sizeof(int2)));
            dev_tab = static_cast<int2 *>(p);
            tab_cap = K;
        }
        host_tab.resize((size_t)K);
        for (int64_t k = 0; k < K; ++k) {
            const int64_t c = k / (KH * KW), r = k % (KH * KW), kh = r / KW, kw = r % KW;
            host_tab[(size_t)k] = make_int2((int)(c * H * W + kh * W + kw), (int)((kh << 16) | kw));
        }
        CAMEL_RETURN_IF(check_hip(hipMemcpyAsync(dev_tab, host_tab.data(), (size_t)K * sizeof(int2),
                                                 hipMemcpyHostToDevice, stream()),
                                  "hipMemcpyAsync(conv table)"));
        CAMEL_RETURN_IF(check_hip(hipStreamSynchronize(stream()), "hipStreamSynchronize"));
        tab_key[0] = C;
        tab_key[1] = KH;
        tab_key[2] = KW;
        tab_key[3] = H * W * 65536 + W;
    }
    GemmArgs g = conv_args(w, x, bias, y, N, C, H, W, Co, KH, KW, stride, pad, OH, OW, flags);
    g.ktab = dev_tab;
    const bool avec = (K % 4 == 0) && ((uintptr_t)w % 16 == 0);
    int rc;
    if (Co <= 64)
        rc = avec ? run_gemm<TileGather64, LOAD_VEC, LOAD_CONV>(g, 1, "conv2d_igemm_kernel")
                  : run_gemm<TileGather64, LOAD_SCALAR, LOAD_CONV>(g, 1, "conv2d_igemm_kernel");
    else
        rc = avec ? run_gemm<TileGather, LOAD_VEC, LOAD_CONV>(g, 1, "conv2d_igemm_kernel")
                  : run_gemm<TileGather, LOAD_SCALAR, LOAD_CONV>(g, 1, "conv2d_igemm_kernel");
    CAMEL_RETURN_IF(rc);
    return ok();
}

// Shared argument checks of the conv2d entry points.
int conv_check(const float *x, const float *w, const float *bias, const float *y, int64_t N,
               int64_t C, int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW, int64_t stride,
               int64_t pad, int flags, const char *what) {
    const std::string name(what);
    if (N < 0 || C <= 0 || H <= 0 || W <= 0 || Co <= 0 || KH <= 0 || KW <= 0 || stride <= 0 ||
        pad < 0)
        return fail(CAMEL_HIP_ERR_SHAPE, name + ": invalid geometry");
    // Each extent fits 32 bits, so the sums below cannot overflow; the
    // products are taken with overflow checks.
    if (N > INT32_MAX || C > INT32_MAX || H > INT32_MAX || W > INT32_MAX || Co > INT32_MAX ||
        stride > INT32_MAX || pad > INT32_MAX)
        return fail(CAMEL_HIP_ERR_SHAPE, name + ": tensor too large");
    if (H + 2 * pad < KH || W + 2 * pad < KW)
        return fail(CAMEL_HIP_ERR_SHAPE, name + ": kernel larger than padded input");
    if (KH > 0xffff || KW > 0xffff) return fail(CAMEL_HIP_ERR_SHAPE, name + ": kernel too large");
    const int64_t OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    if (!product_fits({N, C, H, W}) || !product_fits({N, OH, OW}) ||
        !product_fits({N, Co, OH, OW}) || !product_fits({Co, C, KH, KW}))
        return fail(CAMEL_HIP_ERR_SHAPE, name + ": tensor too large");
    if (flags & ~(CAMEL_EPI_BIAS | CAMEL_EPI_RELU | CAMEL_CONV_X_NHWC | CAMEL_CONV_Y_NHWC |
                  CAMEL_CONV_W_PACKED | CAMEL_CONV_X_NCHW4 | CAMEL_CONV_Y_NCHW4))
        return fail(CAMEL_HIP_ERR_ARG, name + ": unknown flags");
    if ((flags & CAMEL_CONV_X_NHWC) && (flags & CAMEL_CONV_X_NCHW4))
        return fail(CAMEL_HIP_ERR_ARG, name + ": two input layouts");
    if ((flags & CAMEL_CONV_Y_NHWC) && (flags & CAMEL_CONV_Y_NCHW4))
        return fail(CAMEL_HIP_ERR_ARG, name + ": two output layouts");
    if ((flags & CAMEL_CONV_X_NCHW4) && (C % 4 != 0 || ((uintptr_t)x & 15) != 0))
        return fail(CAMEL_HIP_ERR_ARG, name + ": an NCHW4 input needs C % 4 == 0 and 16-byte alignment");
    if ((flags & CAMEL_CONV_Y_NCHW4) && (Co % 4 != 0 || ((uintptr_t)y & 15) != 0))
        return fail(CAMEL_HIP_ERR_ARG, name + ": an NCHW4 output needs Co % 4 == 0 and 16-byte alignment");
    if ((flags & CAMEL_EPI_BIAS) && !bias) return fail(CAMEL_HIP_ERR_ARG, name + ": null bias");
    if (N > 0 && (!x || !w || !y)) return fail(CAMEL_HIP_ERR_ARG, name + ": null operand");
    return CAMEL_HIP_OK;
}

// Every conv2d runs here.  The NHWC implicit GEMM serves C % 16 == 0 and
// reads an NHWC or NCHW4 input in place; the direct kernel serves
// C*KH*KW <= 32 and writes NHWC or NCHW4 directly; every other layout
// combination goes through conversions into pooled scratch, so all of them
// compute the same values.  pool: y is the 2x2 stride-2 max pool of the
// result (from the GEMM epilogue when the NHWC GEMM serves the shape, else a
// pool pass over a scratch result).
int conv2d_run(const float *x, const float *w, const float *bias, float *y, int64_t N, int64_t C,
               int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW, int64_t stride, int64_t pad,
               int flags, bool pool) {
    const int64_t OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    const int64_t K = C * KH * KW, HW = H * W, P = OH * OW;
    const Layout xl = (flags & CAMEL_CONV_X_NHWC)    ? L_NHWC
                      : (flags & CAMEL_CONV_X_NCHW4) ? L_NCHW4
                                                     : L_NCHW;
    const Layout yl = (flags & CAMEL_CONV_Y_NHWC)    ? L_NHWC
                      : (flags & CAMEL_CONV_Y_NCHW4) ? L_NCHW4
                                                     : L_NCHW;
    const int epi = flags & (CAMEL_EPI_BIAS | CAMEL_EPI_RELU);
    const bool aligned = (((uintptr_t)x | (uintptr_t)w) & 15) == 0;
    // (the NCHW -> NHWC transpose runs one image per grid z, plus one z for
    // the weights)
    const bool gemm_nhwc = K > DIRECT_MAX_K && aligned && C % 16 == 0 && N < 65535;
    bool w_packed = (flags & CAMEL_CONV_W_PACKED) != 0;
    Scratch wu;
    if (w_packed && !gemm_nhwc) {
        // the other kernels read w [Co][C][KH][KW]: unpack into scratch
        CAMEL_RETURN_IF(wu.alloc((size_t)(Co * K) * sizeof(float)));
        CAMEL_RETURN_IF(pack_weights(w, wu.f(), Co, KH * KW, C));
        w = wu.f();
        w_packed = false;
        flags &= ~CAMEL_CONV_W_PACKED;
    }
    // out_flags: the epilogue flags, plus CAMEL_CONV_Y_NCHW4 for an NCHW4 out
    auto nhwc_gemm = [&](float *out, bool pooled, int out_flags) -> int {
        const bool k32 = C % 32 == 0;
        if (Co > 64)
            return k32 ? conv2d_nhwc<TileConv>(x, w, bias, out, N, C, H, W, Co, KH, KW, stride, pad, OH,
                                              OW, out_flags, xl, pooled, w_packed)
                       : conv2d_nhwc<TileConv16>(x, w, bias, out, N, C, H, W, Co, KH, KW, stride, pad,
                                                OH, OW, out_flags, xl, pooled, w_packed);
        return k32 ? conv2d_nhwc<TileConv64>(x, w, bias, out, N, C, H, W, Co, KH, KW, stride, pad, OH,
                                            OW, out_flags, xl, pooled, w_packed)
                   : conv2d_nhwc<TileConv64k16>(x, w, bias, out, N, C, H, W, Co, KH, KW, stride, pad,
                                               OH, OW, out_flags, xl, pooled, w_packed);
    };
    if (pool) {
        if (gemm_nhwc) return nhwc_gemm(y, true, epi);
        Scratch full;
        CAMEL_RETURN_IF(full.alloc((size_t)(N * Co * P) * sizeof(float)));
        CAMEL_RETURN_IF(conv2d_run(x, w, bias, full.f(), N, C, H, W, Co, KH, KW, stride, pad,
                                   flags & ~(CAMEL_CONV_Y_NHWC | CAMEL_CONV_Y_NCHW4), false));
        return camel_hip_maxpool2d(full.f(), y, N, Co, OH, OW, 2, 2, 2);
    }
    // The result in y's layout straight from the kernel (NCHW; NCHW4 from
    // the direct kernel and the implicit GEMM; NHWC from the direct kernel),
    // or NCHW into scratch that is then converted.
    const bool direct = K <= DIRECT_MAX_K;
    const bool native_out =
        yl == L_NCHW || (yl == L_NCHW4 && (direct || gemm_nhwc)) ||
        (yl == L_NHWC && direct && Co % 4 == 0 && ((uintptr_t)y & 15) == 0);
    Scratch ytmp;
    float *out = y;
    if (!native_out) {
        CAMEL_RETURN_IF(ytmp.alloc((size_t)(N * Co * P) * sizeof(float)));
        out = ytmp.f();
    }
    if (gemm_nhwc) {
        CAMEL_RETURN_IF(nhwc_gemm(out, false, epi | (out == y && yl == L_NCHW4 ? CAMEL_CONV_Y_NCHW4 : 0)));
    } else {
        Scratch xtmp;
        const float *xs = x;
        if (xl != L_NCHW) {
            CAMEL_RETURN_IF(xtmp.alloc((size_t)(N * C * HW) * sizeof(float)));
            if (xl == L_NHWC)
                CAMEL_RETURN_IF(transpose_images(x, xtmp.f(), N, HW, C));
            else
                CAMEL_RETURN_IF(quad_layout(x, xtmp.f(), N * C / 4, HW, false));
            xs = xtmp.f();
        }
        if (direct)
            CAMEL_RETURN_IF(conv2d_direct(xs, w, bias, out, N, C, H, W, Co, KH, KW, stride, pad, OH, OW,
                                          epi, out == y ? yl : L_NCHW));
        else
            CAMEL_RETURN_IF(conv2d_gather(xs, w, bias, out, N, C, H, W, Co, KH, KW, stride, pad, OH, OW,
                                          epi));
    }
    if (out != y) {
        if (yl == L_NHWC)
            CAMEL_RETURN_IF(transpose_images(out, y, N, Co, P));
        else
            CAMEL_RETURN_IF(quad_layout(out, y, N * Co / 4, P, true));
    }
    return CAMEL_HIP_OK;
}

// Argument checks of the sgemm entry points (before any device work).
int sgemm_check(const float *A, const float *B, const float *C, int64_t M, int64_t N, int64_t K,
                const float *bias, int flags, const char *name) {
    const std::string who(name);
    if (flags & ~(CAMEL_EPI_BIAS | CAMEL_EPI_RELU | CAMEL_GEMM_A_T))
        return fail(CAMEL_HIP_ERR_ARG, who + ": unknown flags");
    if (M < 0 || N < 0 || K < 0) return fail(CAMEL_HIP_ERR_SHAPE, who + ": negative dimension");
    if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2)
        return fail(CAMEL_HIP_ERR_SHAPE, who + ": dimension too large");
    if ((flags & CAMEL_EPI_BIAS) && !bias) return fail(CAMEL_HIP_ERR_ARG, who + ": null bias");
    if (M == 0 || N == 0) return CAMEL_HIP_OK;
    if (!C || (K > 0 && (!A || !B))) return fail(CAMEL_HIP_ERR_ARG, who + ": null operand");
    return CAMEL_HIP_OK;
}

GemmArgs sgemm_args(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K,
                    const float *bias, int flags) {
    GemmArgs g{};
    g.A = A;
    g.B = B;
    g.C = C;
    g.bias = bias;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.lda = (flags & CAMEL_GEMM_A_T) ? (int)M : (int)K;
    g.ldb = (int)N;
    g.ldc = (int)N;
    g.flags = flags & (CAMEL_EPI_BIAS | CAMEL_EPI_RELU);
    return g;
}

// The kernels camel_hip_sgemm runs for a problem, and the bytes of split-K
// partial sums they need (0 when nothing is split).
enum class SgemmPath { Thin, Skinny, Tiles };
struct SgemmPlan {
    SgemmPath path;
    Cfg cfg;
    int splits;
    bool avec, bvec, atrans;
    size_t partial_bytes;
};

// atrans: A is given transposed (CAMEL_GEMM_A_T); only the tile kernel has
// the transposed loaders, so the thin and skinny kernels are not used.
SgemmPlan plan_sgemm(const GemmArgs &g, bool atrans) {
    SgemmPlan p{SgemmPath::Tiles, Cfg::Big, 1, false, false, atrans, 0};
    if (!atrans && thin_eligible(g.M, g.N, g.K)) {
        p.path = SgemmPath::Thin;
        return p;
    }
    if (!atrans && skinny_eligible(g.M, g.N, g.K, g.B, g.C)) {
        p.path = SgemmPath::Skinny;
        p.partial_bytes = skinny_partial_bytes(g.M, g.N, g.K);
        return p;
    }
    p.avec = ((atrans ? g.M : g.K) % 4 == 0) && ((uintptr_t)g.A % 16 == 0);
    p.bvec = (g.N % 4 == 0) && ((uintptr_t)g.B % 16 == 0);
    int bk = 0;
    const int cus = device_cu_count();
    choose(g.M, g.N, g.K, cus, p.cfg, p.splits, bk);
    if (p.cfg == Cfg::Mid && !atrans && p.avec && p.bvec && tiles_of<TileMid>(g.M, g.N) < 2 * cus)
        p.cfg = Cfg::MidK;
    switch (p.cfg) {
    case Cfg::Big:
        p.partial_bytes = gemm_modes_partial_bytes<TileBig>(g, p.splits, p.avec, p.bvec, atrans);
        break;
    case Cfg::Mid:
        p.partial_bytes = gemm_modes_partial_bytes<TileMid>(g, p.splits, p.avec, p.bvec, atrans);
        break;
    case Cfg::MidK:
        p.partial_bytes = gemm_modes_partial_bytes<TileMidK>(g, p.splits, p.avec, p.bvec, atrans);
        break;
    case Cfg::Tiny:
        p.partial_bytes = gemm_modes_partial_bytes<TileTiny>(g, p.splits, p.avec, p.bvec, atrans);
        break;
    case Cfg::Small:
        p.partial_bytes = gemm_modes_partial_bytes<TileSmall>(g, p.splits, p.avec, p.bvec, atrans);
        break;
    default:
        p.partial_bytes = gemm_modes_partial_bytes<TileSkinny>(g, p.splits, p.avec, p.bvec, atrans);
        break;
    }
    return p;
}

int run_sgemm(const GemmArgs &g, const SgemmPlan &p) {
    switch (p.path) {
    case SgemmPath::Thin:
        return launch_thin(g.A, g.B, g.C, g.M, g.N, g.K, g.bias, g.flags);
    case SgemmPath::Skinny:
        return launch_skinny(g.A, g.B, g.C, g.M, g.N, g.K, g.bias, g.flags);
    default:
        break;
    }
    switch (p.cfg) {
    case Cfg::Big:
        return launch_gemm_modes<TileBig>(g, p.splits, p.avec, p.bvec, p.atrans);
    case Cfg::Mid:
        return launch_gemm_modes<TileMid>(g, p.splits, p.avec, p.bvec, p.atrans);
    case Cfg::MidK:
        return launch_gemm_modes<TileMidK>(g, p.splits, p.avec, p.bvec, p.atrans);
    case Cfg::Tiny:
        return launch_gemm_modes<TileTiny>(g, p.splits, p.avec, p.bvec, p.atrans);
    case Cfg::Small:
        return launch_gemm_modes<TileSmall>(g, p.splits, p.avec, p.bvec, p.atrans);
    default:
        return launch_gemm_modes<TileSkinny>(g, p.splits, p.avec, p.bvec, p.atrans);
    }
}

} // namespace
} // namespace camel_hip

using namespace camel_hip;

extern "C" {

int camel_hip_sgemm(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K,
                    const float *bias, int flags) {
    CAMEL_RETURN_IF(sgemm_check(A, B, C, M, N, K, bias, flags, "sgemm"));
    if (M == 0 || N == 0) return ok();
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    const GemmArgs g = sgemm_args(A, B, C, M, N, K, bias, flags);
    CAMEL_RETURN_IF(run_sgemm(g, plan_sgemm(g, (flags & CAMEL_GEMM_A_T) != 0)));
    return ok();
}

int camel_hip_sgemm_noalloc(const float *A, const float *B, float *C, int64_t M, int64_t N,
                            int64_t K, const float *bias, int flags) {
    CAMEL_RETURN_IF(sgemm_check(A, B, C, M, N, K, bias, flags, "sgemm_noalloc"));
    if (M == 0 || N == 0) return ok();
    CAMEL_LOCK();
    // Initialisation allocates (stream, error flag): it belongs to set-up.
    if (!initialised())
        return fail(CAMEL_HIP_ERR_ARG, "sgemm_noalloc: call camel_hip_init before this entry point");
    float *scratch = noalloc_scratch();
    if (!scratch) return fail(CAMEL_HIP_ERR_RUNTIME, "sgemm_noalloc: static scratch not set up");
    const GemmArgs g = sgemm_args(A, B, C, M, N, K, bias, flags);
    const SgemmPlan plan = plan_sgemm(g, (flags & CAMEL_GEMM_A_T) != 0);
    if (plan.partial_bytes > CAMEL_HIP_NOALLOC_SCRATCH_BYTES)
        return fail(CAMEL_HIP_ERR_SHAPE,
                    "sgemm_noalloc: this shape needs " + std::to_string(plan.partial_bytes) +
                        " bytes of split-K scratch, more than the " +
                        std::to_string((size_t)CAMEL_HIP_NOALLOC_SCRATCH_BYTES) +
                        "-byte static scratch");
    FixedPartials fixed(scratch, CAMEL_HIP_NOALLOC_SCRATCH_BYTES);
    CAMEL_RETURN_IF(run_sgemm(g, plan));
    return ok();
}

int camel_hip_dense_softmax(const float *A, const float *B, const float *bias, float *C, int64_t M,
                            int64_t N, int64_t K, int flags) {
    if (M < 0 || N < 0 || K < 0) return fail(CAMEL_HIP_ERR_SHAPE, "dense_softmax: negative dimension");
    if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2)
        return fail(CAMEL_HIP_ERR_SHAPE, "dense_softmax: dimension too large");
    if ((flags & CAMEL_EPI_BIAS) && !bias) return fail(CAMEL_HIP_ERR_ARG, "dense_softmax: null bias");
    if (M == 0 || N == 0) return ok();
    if (!C || (K > 0 && (!A || !B))) return fail(CAMEL_HIP_ERR_ARG, "dense_softmax: null operand");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    if (thin_eligible(M, N, K)) {
        CAMEL_RETURN_IF(launch_thin<true>(A, B, C, (int)M, (int)N, (int)K, bias, flags));
        return ok();
    }
    // Unfused: the GEMM with its epilogue, then the row softmax in place
    // (each row is read whole before it is written).
    CAMEL_RETURN_IF(camel_hip_sgemm(A, B, C, M, N, K, bias, flags));
    CAMEL_RETURN_IF(camel_hip_softmax_rows(C, C, M, N));
    return ok();
}

int camel_hip_dense_head(const float *x, const float *w1, const float *b1, const float *w2,
                         const float *b2, float *y, int64_t M, int64_t K1, int64_t N1, int64_t N2,
                         int flags1, int flags2, int softmax) {
    if (M < 0 || K1 < 0 || N1 < 0 || N2 < 0)
        return fail(CAMEL_HIP_ERR_SHAPE, "dense_head: negative dimension");
    if (M > INT32_MAX / 2 || K1 > INT32_MAX / 2 || N1 > INT32_MAX / 2 || N2 > INT32_MAX / 2)
        return fail(CAMEL_HIP_ERR_SHAPE, "dense_head: dimension too large");
    if (((flags1 & CAMEL_EPI_BIAS) && !b1) || ((flags2 & CAMEL_EPI_BIAS) && !b2))
        return fail(CAMEL_HIP_ERR_ARG, "dense_head: null bias");
    if ((flags1 | flags2) & ~(CAMEL_EPI_BIAS | CAMEL_EPI_RELU))
        return fail(CAMEL_HIP_ERR_ARG, "dense_head: unknown flags");
    if (M == 0 || N2 == 0) return ok();
    if (!y || (K1 > 0 && (!x || !w1)) || (N1 > 0 && !w2))
        return fail(CAMEL_HIP_ERR_ARG, "dense_head: null operand");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    // Fused when layer 1 runs as a split-K GEMM of the main kernel and layer
    // 2 as the 16-wave thin kernel: the thin kernel rebuilds layer 1's rows
    // from the partials (no reduce launch, no intermediate in HBM).
    Cfg cfg = Cfg::Skinny;
    int splits = 1, bk = 0;
    if (N2 <= 16 && thin_eligible(M, N2, N1) && !thin_eligible(M, N1, K1) && M > 32)
        choose(M, N1, K1, device_cu_count(), cfg, splits, bk);
    const bool avec = (K1 % 4 == 0) && ((uintptr_t)x % 16 == 0);
    const bool bvec = (N1 % 4 == 0) && ((uintptr_t)w1 % 16 == 0);
    if (cfg == Cfg::Small && splits <= 1 && avec && bvec && M % TileSmall::BM == 0 &&
        N1 % TileSmall::BN == 0 && N1 <= (int64_t)HEAD_MAX_N2 * TileSmall::BN &&
        N2 <= HEAD_MAX_N2 && M <= INT32_MAX / HEAD_MAX_N2) {
        // Layer 1 runs unsplit on 64 x 64 tiles (e.g. the MLP's 1024 x 1024
        // -> 1024): each tile's epilogue multiplies its finished 64 columns
        // by their 64 rows of w2, and head_finish_kernel adds the tiles' sums
        // in tile order -- layer 1's output never reaches HBM and the thin
        // kernel's staging of w2 is not needed.
        const int tiles_m = (int)(M / TileSmall::BM), tiles_n = (int)(N1 / TileSmall::BN);
        Scratch part;
        CAMEL_RETURN_IF(part.alloc((size_t)tiles_n * M * N2 * sizeof(float)));
        GemmArgs g = sgemm_args(x, w1, nullptr, M, N1, K1, b1, flags1);
        g.head_w = w2;
        g.head_partial = part.f();
        g.head_n2 = (int)N2;
        if (dma_eligible<TileSmall>(g, avec, bvec))
            CAMEL_RETURN_IF((launch_range<TileSmall, LOAD_DMA, LOAD_DMA>(g, 0, tiles_m * tiles_n, 1,
                                                                          "sgemm_kernel")));
        else
            CAMEL_RETURN_IF((launch_range<TileSmall, LOAD_VEC, LOAD_VEC>(g, 0, tiles_m * tiles_n, 1,
                                                                          "sgemm_kernel")));
        const unsigned blocks = (unsigned)((M + 3) / 4);
        if (softmax)
            hipLaunchKernelGGL(head_finish_kernel<true>, dim3(blocks), dim3(256), 0, stream(), part.f(),
                               tiles_n, (int)M, (int)N2, b2, flags2, y);
        else
            hipLaunchKernelGGL(head_finish_kernel<false>, dim3(blocks), dim3(256), 0, stream(),
                               part.f(), tiles_n, (int)M, (int)N2, b2, flags2, y);
        CAMEL_RETURN_IF(check_launch("head_finish_kernel"));
        return ok();
    }
    if (cfg == Cfg::Skinny || splits <= 1) {
        Scratch h;
        CAMEL_RETURN_IF(h.alloc((size_t)(M * N1) * sizeof(float)));
        CAMEL_RETURN_IF(camel_hip_sgemm(x, w1, h.f(), M, N1, K1, b1, flags1));
        if (softmax) return camel_hip_dense_softmax(h.f(), w2, b2, y, M, N2, N1, flags2);
        return camel_hip_sgemm(h.f(), w2, y, M, N2, N1, b2, flags2);
    }
    GemmArgs g{};
    g.A = x;
    g.B = w1;
    g.C = y; // not written: the launch leaves partials
    g.bias = b1;
    g.M = (int)M;
    g.N = (int)N1;
    g.K = (int)K1;
    g.lda = (int)K1;
    g.ldb = (int)N1;
    g.ldc = (int)N1;
    g.flags = flags1;
    SplitPartialsA src{};
    switch (cfg) {
    case Cfg::Big:
        CAMEL_RETURN_IF(launch_split_partials<TileBig>(g, splits, avec, bvec, src));
        break;
    case Cfg::Mid:
        CAMEL_RETURN_IF(launch_split_partials<TileMid>(g, splits, avec, bvec, src));
        break;
    case Cfg::Tiny:
        CAMEL_RETURN_IF(launch_split_partials<TileTiny>(g, splits, avec, bvec, src));
        break;
    default:
        CAMEL_RETURN_IF(launch_split_partials<TileSmall>(g, splits, avec, bvec, src));
        break;
    }
    if (softmax)
        CAMEL_RETURN_IF((launch_thin_rows<true>(src, w2, y, (int)M, (int)N2, (int)N1, b2, flags2)));
    else
        CAMEL_RETURN_IF((launch_thin_rows<false>(src, w2, y, (int)M, (int)N2, (int)N1, b2, flags2)));
    return ok();
}

int camel_hip_matmul_generic(int adt, const void *A, int bdt, const void *B, int odt, void *C,
                             int64_t M, int64_t N, int64_t K) {
    if (!valid_dtype(adt) || !valid_dtype(bdt) || !valid_dtype(odt))
        return fail(CAMEL_HIP_ERR_DTYPE, "matmul: unsupported dtype");
    if (M < 0 || N < 0 || K < 0) return fail(CAMEL_HIP_ERR_SHAPE, "matmul: negative dimension");
    // Element offsets are int64 in the kernel; every operand's byte count
    // must fit too (8-byte elements at most).
    if (!product_fits({M, K, 8}, INT64_MAX) || !product_fits({K, N, 8}, INT64_MAX) ||
        !product_fits({M, N, 8}, INT64_MAX))
        return fail(CAMEL_HIP_ERR_SHAPE, "matmul: tensor too large");
    if (M == 0 || N == 0) return ok();
    if (!C || (K > 0 && (!A || !B))) return fail(CAMEL_HIP_ERR_ARG, "matmul: null operand");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    hipLaunchKernelGGL(matmul_generic_kernel, dim3(grid_for(M * N, 256)), dim3(256), 0, stream(),
                       adt, A, bdt, B, odt, C, M, N, K);
    CAMEL_RETURN_IF(check_launch("matmul_generic_kernel"));
    return ok();
}

int camel_hip_conv2d(const float *x, const float *w, const float *bias, float *y, int64_t N,
                     int64_t C, int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW,
                     int64_t stride, int64_t pad, int flags) {
    CAMEL_RETURN_IF(conv_check(x, w, bias, y, N, C, H, W, Co, KH, KW, stride, pad, flags, "conv2d"));
    if (N == 0) return ok();
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    CAMEL_RETURN_IF(conv2d_run(x, w, bias, y, N, C, H, W, Co, KH, KW, stride, pad, flags, false));
    return ok();
}

int camel_hip_conv2d_pack_weights(const float *w, float *wp, int64_t Co, int64_t C, int64_t KH,
                                  int64_t KW) {
    if (Co < 0 || C < 0 || KH < 0 || KW < 0) return fail(CAMEL_HIP_ERR_SHAPE, "conv2d_pack_weights: negative dimension");
    if (!product_fits({Co, C, KH, KW}))
        return fail(CAMEL_HIP_ERR_SHAPE, "conv2d_pack_weights: tensor too large");
    if (Co * C * KH * KW == 0) return ok();
    if (!w || !wp) return fail(CAMEL_HIP_ERR_ARG, "conv2d_pack_weights: null pointer");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    CAMEL_RETURN_IF(pack_weights(w, wp, Co, C, KH * KW));
    return ok();
}

int camel_hip_conv2d_pair_pool2(const float *x, const float *w1, const float *b1, const float *w2,
                                const float *b2, float *y, int64_t N, int64_t H, int64_t W,
                                int64_t C1, int64_t Co2, int flags1, int flags2) {
    const char *who = "conv2d_pair_pool2";
    if (N < 0 || H <= 0 || W <= 0 || C1 <= 0 || Co2 <= 0)
        return fail(CAMEL_HIP_ERR_SHAPE, std::string(who) + ": invalid geometry");
    if ((flags1 & ~(CAMEL_EPI_BIAS | CAMEL_EPI_RELU)) ||
        (flags2 & ~(CAMEL_EPI_BIAS | CAMEL_EPI_RELU | CAMEL_CONV_W_PACKED)))
        return fail(CAMEL_HIP_ERR_ARG, std::string(who) + ": unknown flags");
    if (!conv_pair_supported(H, W, C1, Co2) || N > INT32_MAX / 64 ||
        !product_fits({N, Co2, (H - 4) / 2, (W - 4) / 2}))
        return fail(CAMEL_HIP_ERR_SHAPE,
                    std::string(who) + ": shape not served (needs W = 28, C1 = 32, Co2 % 64 == 0, "
                                       "(H - 4) % 8 == 0)");
    if (((flags1 & CAMEL_EPI_BIAS) && !b1) || ((flags2 & CAMEL_EPI_BIAS) && !b2))
        return fail(CAMEL_HIP_ERR_ARG, std::string(who) + ": null bias");
    if (N == 0) return ok();
    if (!x || !w1 || !w2 || !y) return fail(CAMEL_HIP_ERR_ARG, std::string(who) + ": null operand");
    if ((((uintptr_t)w2 | (uintptr_t)x) & 15) != 0)
        return fail(CAMEL_HIP_ERR_ARG, std::string(who) + ": x and w2 must be 16-byte aligned");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    const float *w2p = w2;
    Scratch packed;
    if (!(flags2 & CAMEL_CONV_W_PACKED)) {
        CAMEL_RETURN_IF(packed.alloc((size_t)Co2 * C1 * 9 * sizeof(float)));
        CAMEL_RETURN_IF(pack_weights(w2, packed.f(), Co2, C1, 9));
        w2p = packed.f();
    }
    const int bands = (int)((H - 4) / 2 / CP_BR);
    const dim3 grid((unsigned)(N * bands), (unsigned)(Co2 / 64));
    hipLaunchKernelGGL(conv_pair_pool_kernel, grid, dim3(256), 0, stream(), x, w1, b1, w2p, b2, y,
                       (int)H, (int)Co2, bands, flags1 & (CAMEL_EPI_BIAS | CAMEL_EPI_RELU),
                       flags2 & (CAMEL_EPI_BIAS | CAMEL_EPI_RELU));
    const int rc = check_launch("conv_pair_pool_kernel");
    CAMEL_RETURN_IF(rc);
    return ok();
}

int camel_hip_conv2d_pool2(const float *x, const float *w, const float *bias, float *y, int64_t N,
                           int64_t C, int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW,
                           int64_t stride, int64_t pad, int flags) {
    CAMEL_RETURN_IF(
        conv_check(x, w, bias, y, N, C, H, W, Co, KH, KW, stride, pad, flags, "conv2d_pool2"));
    if (flags & (CAMEL_CONV_Y_NHWC | CAMEL_CONV_Y_NCHW4))
        return fail(CAMEL_HIP_ERR_ARG, "conv2d_pool2: the pooled output is NCHW only");
    const int64_t OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    if (OH < 2 || OW < 2) return fail(CAMEL_HIP_ERR_SHAPE, "conv2d_pool2: window larger than input");
    if (N == 0) return ok();
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    CAMEL_RETURN_IF(conv2d_run(x, w, bias, y, N, C, H, W, Co, KH, KW, stride, pad, flags, true));
    return ok();
}

} // extern "C"
