// sk_abi.hip - extern "C" entry points of libstarter_amd.so (declared in
// include/starter_amd.h): argument validation, the launch planner and the
// kernel launches.  Validation happens before any HIP call, so a rejected
// call touches neither the device nor the stream.
#include "starter_amd.h"

#include <hip/hip_runtime.h>

#include <mutex>
#include <string.h>
#include <unordered_map>

#define SK_AUX_KERNELS 1
#include "sk_registry.hpp"

// Device scratch of sk_gemm_bf16_noalloc: split-K arrival counters and fp32
// partials, SK_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.
// In host code this name is only a stand-in: kernels get the device address
// from hipGetSymbolAddress (scratch_address below), never the name itself.
static __device__ __align__(256) unsigned char scratch[SK_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kDefaultCU = 256;          // MI355X compute units
constexpr int kMaxGrid = 8192;           // bound on workgroups of a persistent launch
constexpr size_t kMaxLds = 160 * 1024;   // gfx950 LDS per CU (dynamic LDS budget per workgroup)
constexpr size_t kPrefLds = 64 * 1024;   // keep >= 2 workgroups per CU when the table has a choice
constexpr int kArgmaxChunk = 4096;       // columns per workgroup of sk_argmax_bf16
constexpr int kMaxM = 64;                // rows of a launch without row groups, and of one row group
constexpr int kMaxLaunchM = 128;         // rows of a launch with row groups; more are chunked

int cdiv(int a, int b) { return (a + b - 1) / b; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Device facts, queried once per device.
// ---------------------------------------------------------------------------
struct DevInfo {
  int status = -1;   // -1 unknown, else sk_status
  int num_cu = 0;
};

std::mutex g_mu;
DevInfo g_dev[64];

int device_info(int* num_cu) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return SK_ERR_DEVICE;
  std::lock_guard<std::mutex> lk(g_mu);
  DevInfo& d = g_dev[dev];
  if (d.status < 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      d.status = SK_ERR_DEVICE;
    } else if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
      d.status = SK_ERR_DEVICE;   // code objects are built for gfx950 only
    } else {
      d.num_cu = prop.multiProcessorCount;
      d.status = SK_OK;
    }
  }
  *num_cu = d.num_cu;
  return d.status;
}

// Occupancy (workgroups per CU) and static limits of a kernel instance.
struct FnInfo {
  int max_threads = 0;
  size_t spill = 0;
};
std::unordered_map<const void*, FnInfo> g_fn;
std::unordered_map<unsigned long long, int> g_occ;

int fn_info(const void* fn, FnInfo* out) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_fn.find(fn);
  if (it == g_fn.end()) {
    hipFuncAttributes a;
    if (hipFuncGetAttributes(&a, fn) != hipSuccess) return SK_ERR_DEVICE;
    FnInfo f;
    f.max_threads = a.maxThreadsPerBlock;
    f.spill = a.localSizeBytes;
    it = g_fn.emplace(fn, f).first;
  }
  *out = it->second;
  return SK_OK;
}

int occupancy(const void* fn, int threads, size_t lds) {
  const unsigned long long key =
      (reinterpret_cast<uintptr_t>(fn) * 1315423911ull) ^ ((unsigned long long)threads << 40) ^ (unsigned long long)lds;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_occ.find(key);
    if (it != g_occ.end()) return it->second;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn), threads, lds) != hipSuccess)
    n = 1;
  if (n < 1) n = 1;
  std::lock_guard<std::mutex> lk(g_mu);
  g_occ[key] = n;
  return n;
}

// ---------------------------------------------------------------------------
// Planner: config -> kernel instance, decomposition, LDS and workspace.
// ---------------------------------------------------------------------------
struct Plan {
  sk_config cfg;
  int epi = 0;
  int tm = 0, tn = 0, tku = 0;  // template parameters: MT|MR, NT|R, KU bound
  int nrb = 0;                  // tiles along N
  int slice_units = 0;
  int out_rows = 0;             // staged output columns per tile (the kernel's OUT_ROWS)
  int tr = 0;                   // output columns per tile (<= out_rows; fewer on the ring path)
  size_t pre_lds = 0;           // per-wave weight staging (LDS-transposed MFMA path)
  size_t parts_lds = 0;         // fp32 partial tiles (pbuf buffers)
  int pbuf = 2;                 // partial tile buffers (1 only on the ring path when 2 do not fit)
  int groups = 1;               // row groups (sk_config::groups), each planned for `mrows` rows
  int mrows = 0;
  size_t stage_elem = 0;        // LDS bytes per staged tile (0: argmax keeps 8*M bytes)
  size_t lds = 0;               // total dynamic LDS (set once the grid is known)
  bool norm = false;            // the op has the add + RMSNorm prologue
  bool fused = false;           // ... and it runs inside the projection kernel
  sk::KernelFn fn = nullptr;
};

bool is_norm_op(int op) {
  return op == SK_OP_RMSNORM_GEMM || op == SK_OP_RMSNORM_GATEUP || op == SK_OP_RMSNORM_LM_ARGMAX;
}
// The projection an op performs (the norm ops map to GEMM / GATEUP / LM_ARGMAX).
int base_op(int op) { return is_norm_op(op) ? op - SK_OP_RMSNORM_GEMM : op; }
bool is_gemm_family(int op) { return op == SK_OP_GEMM || op == SK_OP_GATEUP || op == SK_OP_LM_ARGMAX; }

// The epilogue proper of an instance's epilogue id (the norm-prologue ids
// 5..7 and the residual hand-off consumers 8..10 share the layout of 0..2;
// the hand-off producers 11 and 12 that of STORE and PART).
int epi_base(int epi) {
  if (epi >= sk::EPI_STORE_NORM && epi <= sk::EPI_ARGMAX_NORM) return epi - sk::EPI_STORE_NORM;
  if (epi >= sk::EPI_STORE_PRE && epi <= sk::EPI_ARGMAX_PRE) return epi - sk::EPI_STORE_PRE;
  if (epi == sk::EPI_STORE_RESID) return sk::EPI_STORE;
  if (epi == sk::EPI_PART_RESID) return sk::EPI_PART;
  return epi;
}

// Staged output bytes per element of each epilogue (see EpiTraits).
size_t stage_bytes(int epi) {
  switch (epi_base(epi)) {
    case sk::EPI_STORE: case sk::EPI_SWIGLU: return 2;
    case sk::EPI_PART: return 4;
    case sk::EPI_PART_GU: return 8;
  }
  return 0;
}

// Dynamic LDS of a plan whose workgroups each own at most tiles_per tiles.
size_t plan_lds(const Plan& pl, int M, int tiles_per) {
  if (epi_base(pl.epi) == sk::EPI_ARGMAX) return pl.pre_lds + pl.parts_lds + 8 * (size_t)M + 16;
  return pl.pre_lds + pl.parts_lds + (size_t)tiles_per * pl.stage_elem;
}

// The compiled instance a plan launches (host-side table code; nullptr when
// that instance is not built).
sk::KernelFn plan_kernel(const Plan& pl) {
  if (pl.cfg.path == SK_PATH_MFMA) return sk::mfma_kernel_for(pl.epi, pl.tm, pl.tn, pl.tku);
  if (pl.cfg.path == SK_PATH_WIDE)
    return sk::wide_kernel_for(pl.epi, pl.cfg.waves, pl.cfg.groups > 1 ? pl.cfg.groups : 1, pl.tn);
  if (pl.cfg.path == SK_PATH_MFMA_LDS)
    return pl.groups > 1 ? sk::mfmt_grouped_kernel_for(pl.epi, pl.tm, pl.tn, pl.tku)
                         : sk::mfmt_kernel_for(pl.epi, pl.tm, pl.tn, pl.tku);
  return sk::gemv_kernel_for(pl.epi, pl.tm, pl.tn, pl.tku);
}

int bucket(const int* list, int n, int v) {
  for (int i = 0; i < n; ++i)
    if (list[i] >= v) return list[i];
  return -1;
}

int epi_for(int op, int split) {
  if (op == SK_OP_GEMM) return split > 1 ? sk::EPI_PART : sk::EPI_STORE;
  if (op == SK_OP_GATEUP) return split > 1 ? sk::EPI_PART_GU : sk::EPI_SWIGLU;
  return sk::EPI_ARGMAX;
}

// Pure host logic: fills everything except fn/grid-from-occupancy.  op is a
// projection (GEMM / GATEUP / LM_ARGMAX); `fused` selects the instances with
// the norm prologue.
// variant: 0 plain, 1 residual hand-off consumer (EPI_*_PRE), 2 producer
// (EPI_*_RESID); both run on the ring-streamed LDS-fed MFMA path or the
// two-operand wide path.
int plan_shape_impl(int op, int M, int N, int K, const sk_config& c, bool fused, Plan* pl, int variant = 0) {
  if (!is_gemm_family(op)) return SK_ERR_CONFIG;
  if (M < 1 || M > kMaxLaunchM || N < 1 || K < 32 || (K & 31) != 0) return SK_ERR_SHAPE;
  if (c.waves < 1 || c.waves > 16 || c.ku < 1 || c.split < 1 || c.grid < 0 || c.groups < 0) return SK_ERR_CONFIG;
  if (op == SK_OP_LM_ARGMAX && c.split != 1) return SK_ERR_CONFIG;
  // Row groups: ring path (no norm prologue), an explicit grid that keeps
  // sibling workgroups on one XCD, and a row in every group; the rest of the
  // plan is that of one group.
  // (the wide path reads `groups` as the wave groups along the tile's weight
  // slabs, not as row groups)
  const int groups = c.groups > 1 && c.path != SK_PATH_WIDE ? c.groups : 1;
  if (groups > 1) {
    if (fused || c.path != SK_PATH_MFMA_LDS || (c.ku != 8 && c.ku != 32)) return SK_ERR_CONFIG;
    if (c.grid <= 0 || (c.grid % 8) != 0) return SK_ERR_CONFIG;
    const int mrows = cdiv(M, groups);
    if ((groups - 1) * mrows >= M) return SK_ERR_CONFIG;
    M = mrows;
  }
  // more rows than an instance holds: chunked, or row groups (the wide path
  // holds up to kMaxLaunchM rows in one workgroup)
  if (M > (c.path == SK_PATH_WIDE && groups == 1 ? kMaxLaunchM : kMaxM)) return SK_ERR_SHAPE;
  pl->groups = groups;
  pl->mrows = M;
  const bool gateup = (op == SK_OP_GATEUP);
  if (fused && (c.split != 1 || c.path != SK_PATH_GEMV)) return SK_ERR_CONFIG;
  if (variant != 0) {
    if (fused) return SK_ERR_CONFIG;
    if (variant == 2 && op != SK_OP_GEMM) return SK_ERR_CONFIG;
    if (c.path == SK_PATH_WIDE) {
      // the two-operand wide body: consumers with one K split (whole 16-column
      // groups of partial sums), the producer after split-K partials (its
      // tiles are whole 16-column groups, checked below)
      if (c.groups != 4) return SK_ERR_CONFIG;
      if (variant == 1 && (c.split != 1 || (K & 15) != 0)) return SK_ERR_CONFIG;
      if (variant == 2 && (c.split < 2 || (c.rows & 15) != 0)) return SK_ERR_CONFIG;
    } else {
      if (c.path != SK_PATH_MFMA_LDS || c.ku == 16) return SK_ERR_CONFIG;
      // consumers: one K split; the prologue loads each wave's share of the
      // partial sums in one pass (rows <= 4 per wave, <= 256 groups per row)
      if (variant == 1 && (c.ku != 8 || c.split != 1 || (K & 15) != 0 || M > 4 * c.waves || K > 4096))
        return SK_ERR_CONFIG;
    }
  }
  pl->cfg = c;
  pl->epi = epi_for(op, c.split) + (fused ? sk::EPI_STORE_NORM : 0);
  if (variant == 1) pl->epi = epi_for(op, c.split) + sk::EPI_STORE_PRE;
  if (variant == 2) pl->epi = c.split > 1 ? sk::EPI_PART_RESID : sk::EPI_STORE_RESID;
  pl->fused = fused;
  int units, partial_rows;
  if (c.path == SK_PATH_MFMA) {
    if (gateup ? c.rows != 16 : (c.rows != 16 && c.rows != 32)) return SK_ERR_CONFIG;
    units = K / 32;
    pl->tm = cdiv(M, 16);
    pl->tn = gateup ? 2 : c.rows / 16;
    pl->tku = bucket(sk::kMfmaKU, (int)(sizeof(sk::kMfmaKU) / sizeof(int)), c.ku);
    partial_rows = 16 * pl->tn;
    if (pl->tku < 0 || c.waves > sk::instance_waves(sk::KIND_MFMA, pl->tm, pl->tn, pl->tku, pl->epi))
      return SK_ERR_CONFIG;
  } else if (c.path == SK_PATH_MFMA_LDS) {
    // One K range of KW = 32*ku columns per wave: 256, 1024 or 1280 (one,
    // four or five 256-column chunks, ring-streamed) or 512 (whole tiles in
    // flight).
    // The ring path takes any tile height up to 32 rows (48 for gate/up):
    // its slabs are 16 rows and the rows past `rows` are not loaded, so a
    // tile of N / 256 rows gives every CU one tile.  The whole-tile body and
    // the residual hand-off take 16 or 32 (gate/up: 16).
    if (c.ku != 8 && c.ku != 16 && c.ku != 32 && c.ku != 40) return SK_ERR_CONFIG;
    const bool any_rows = c.ku != 16 && variant == 0;
    if (any_rows ? (c.rows < 1 || c.rows > (gateup ? 48 : 32))
                 : (gateup ? c.rows != 16 : (c.rows != 16 && c.rows != 32)))
      return SK_ERR_CONFIG;
    const int KW = 32 * c.ku;
    units = cdiv(K, KW);
    pl->tm = cdiv(M, 16);
    pl->tn = gateup ? 2 * cdiv(c.rows, 16) : cdiv(c.rows, 16);
    pl->tku = KW;
    partial_rows = 16 * pl->tn;
    if (c.waves > sk::instance_waves(sk::KIND_MFMT, pl->tm, pl->tn, KW, pl->epi)) return SK_ERR_CONFIG;
    pl->pre_lds = (size_t)c.waves * 16 * (2 * 256 + sk::kRowPad);
  } else if (c.path == SK_PATH_WIDE) {
    // All rows in one workgroup: W = 4 or 8 waves split the (up to 8)
    // 16-row activation tiles, every wave multiplies the whole weight tile
    // of `rows` rows (gate/up: rows gate + rows up), staged in LDS in
    // 256-column steps (ku = 8).
    // `groups` (1 or 2) = WN, the wave groups along the tile's slabs;
    // groups = 4 selects the body that stages the activation rows in LDS too
    // (four waves, two activation tiles each, every wave on the whole tile).
    const int wn = c.groups > 1 ? c.groups : 1;
    if ((variant != 0 && wn != 4) || (wn != 1 && wn != 2 && wn != 4) || (wn == 2 && c.waves != 8)) return SK_ERR_CONFIG;
    if ((c.waves != 4 && c.waves != 8) || c.ku != 8) return SK_ERR_CONFIG;
    const int max_rows = wn == 4 ? (gateup ? 64 : 128) : (gateup ? (wn == 2 ? 32 : 48) : 96);
    if (c.rows < 1 || c.rows > max_rows) return SK_ERR_CONFIG;
    units = cdiv(K, sk::kWideChunk);
    pl->tm = cdiv(M, 16);
    const int half = cdiv(c.rows, 16);                    // slabs per half (gate/up) or per tile
    const int hw = wn == 4 ? half : cdiv(half, wn) * wn;  // rounded to whole slabs per wave group
    pl->tn = gateup ? 2 * hw : hw;
    if (pl->tn < 2) pl->tn = 2;   // the smallest instance stages two slabs
    if (wn == 4 && (pl->tn == 7 || (c.waves == 8 && (pl->tn & 1)))) pl->tn += 1;   // compiled slab counts
    if (variant == 2 && 16 * pl->tn != c.rows) return SK_ERR_CONFIG;   // the finish's 16-column groups
    pl->tku = sk::kWideChunk;
    partial_rows = 0;
    pl->pre_lds = wn == 4 ? sk::wide2_lds(pl->tn) : sk::wide_weight_lds(pl->tn);
  } else if (c.path == SK_PATH_GEMV) {
    if (c.rows != 2 && c.rows != 4 && c.rows != 8) return SK_ERR_CONFIG;
    if (M > 8) return SK_ERR_CONFIG;
    units = cdiv(K, 512);
    pl->tm = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8));
    pl->tn = c.rows;
    pl->tku = bucket(sk::kGemvKU, (int)(sizeof(sk::kGemvKU) / sizeof(int)), c.ku);
    partial_rows = gateup ? 2 * c.rows : c.rows;
    if (pl->tku < 0 || c.waves > sk::instance_waves(sk::KIND_GEMV, pl->tm, pl->tn, pl->tku, pl->epi))
      return SK_ERR_CONFIG;
  } else {
    return SK_ERR_CONFIG;
  }
  if (pl->tku < 0) return SK_ERR_CONFIG;
  // The instance must be compiled (the lookup is host-side table code).
  if (!plan_kernel(*pl)) return SK_ERR_CONFIG;
  pl->slice_units = cdiv(units, c.split);
  const long per_wave = c.path == SK_PATH_MFMA_LDS ? 1 : c.ku;
  // (the wide path's waves all walk the whole slice)
  if (c.path != SK_PATH_WIDE && (long)c.waves * per_wave < pl->slice_units) return SK_ERR_CONFIG;   // K slice not covered
  if (c.split > 1 && (c.split - 1) * pl->slice_units >= units) return SK_ERR_CONFIG;  // empty split
  const bool lds_fed = c.path == SK_PATH_MFMA_LDS || c.path == SK_PATH_WIDE;
  const int out_rows = c.path == SK_PATH_MFMA ? (gateup ? 16 : c.rows)
                       : lds_fed             ? (gateup ? 8 * pl->tn : 16 * pl->tn)
                                             : c.rows;
  pl->out_rows = out_rows;
  pl->tr = lds_fed ? c.rows : out_rows;
  pl->nrb = cdiv(N, pl->tr);
  if (c.path == SK_PATH_MFMA_LDS) partial_rows = sk::lds_part_stride(pl->tm, pl->tn, pl->tku);
  pl->parts_lds = (size_t)2 * c.waves * M * partial_rows * sizeof(float);
  pl->stage_elem = stage_bytes(pl->epi) * (size_t)M * out_rows;
  if (c.path == SK_PATH_WIDE) {   // outputs go straight from registers; the split-K finish's flags
    pl->parts_lds = (size_t)64 * c.waves * sizeof(int);
    pl->stage_elem = 0;
  }
  if (c.grid > 0 && (c.grid % c.split) != 0) return SK_ERR_CONFIG;
  const int tiles_per = c.grid > 0 ? cdiv(pl->nrb, c.grid / c.split) : 1;
  pl->lds = plan_lds(*pl, M, tiles_per);
  // The ring path can work with one partial tile buffer (one more barrier per
  // tile) where two would not fit.
  const bool ring = c.path == SK_PATH_MFMA_LDS && pl->tku != 512;   // (not the wide path)
  if (ring && (pl->lds > kMaxLds || (c.grid == 0 && plan_lds(*pl, M, cdiv(pl->nrb, kMaxGrid)) > kMaxLds))) {
    pl->pbuf = 1;
    pl->parts_lds /= 2;
    pl->lds = plan_lds(*pl, M, tiles_per);
  }
  if (pl->lds > kMaxLds) return SK_ERR_CONFIG;
  // A derived grid holds at most kMaxGrid workgroups per K split, so every
  // workgroup may have to stage cdiv(nrb, kMaxGrid) tiles.
  if (c.grid == 0 && plan_lds(*pl, M, cdiv(pl->nrb, kMaxGrid)) > kMaxLds) return SK_ERR_CONFIG;
  return SK_OK;
}

// Plan of any GEMM-family op.  A norm op runs its prologue inside the
// projection kernel on the GEMV path with one K split (a compiled norm
// instance within the wave limit), else as a separate add+norm launch in
// front of the plain projection.  The MFMA paths take the separate launch:
// there every workgroup would normalise the whole activation block again,
// and on an MI355X that VALU work cost more than the extra launch (qkv at
// M = 16: 16.5 us fused in the LDS-fed MFMA kernel, 12.6 us as two launches).
int plan_shape(int op, int M, int N, int K, const sk_config& c, Plan* pl) {
  const bool norm = is_norm_op(op);
  const int bop = base_op(op);
  if (norm && c.split == 1 && c.path == SK_PATH_GEMV && plan_shape_impl(bop, M, N, K, c, true, pl) == SK_OK) {
    pl->norm = true;
    return SK_OK;
  }
  const int st = plan_shape_impl(bop, M, N, K, c, false, pl);
  pl->norm = norm;
  return st;
}

// Upper bound of the workgroups a plan launches (what the workspace covers).
int grid_bound(const Plan& pl) {
  if (pl.cfg.grid > 0) return pl.cfg.grid;
  return pl.cfg.split * (pl.nrb < kMaxGrid ? pl.nrb : kMaxGrid);
}

// Workspace layout: [arrival counters, padded to 256 B][partials or argmax
// candidates].  The counters must be zero before the first call (allocate the
// workspace zero-filled); every call returns them to zero.
size_t ticket_bytes(int n) { return (((size_t)n * sizeof(unsigned)) + 255) & ~(size_t)255; }

// With row groups: one counter (argmax) or one per tile for each group, the
// argmax candidates of all M rows, and one partials region per group.
size_t plan_tickets(int op, const Plan& pl) {
  return ticket_bytes(pl.groups * (base_op(op) == SK_OP_LM_ARGMAX ? 1 : pl.nrb));
}
size_t plan_workspace(int op, int M, int N, const Plan& pl) {
  op = base_op(op);
  if (op == SK_OP_LM_ARGMAX) return plan_tickets(op, pl) + (size_t)M * sizeof(unsigned long long);
  if (pl.cfg.split > 1)
    return plan_tickets(op, pl) +
           (size_t)pl.groups * (op == SK_OP_GATEUP ? 2 : 1) * pl.cfg.split * pl.mrows * (size_t)N * sizeof(float);
  return 0;
}

// Offline-tuned launch table for the Qwen3-4B decode shapes (the reference
// picks a Triton config per shape at warmup: engine/kernels/gemm.py:516-660).
// Each entry is the fastest configuration measured on one MI355X for that
// shape at that row count, timed as graph replays of back-to-back launches
// over 24 distinct weight copies (so HBM, not the 256 MB MALL, serves the
// weights).  Fields: {path, waves, ku, rows, split, grid, groups}.
struct Tuned {
  int op, N, K, M;
  sk_config cfg;
};

const Tuned kTuned[] = {
    {SK_OP_GEMM, 6144, 2560, 1, {2, 1, 5, 2, 1, 0}},  // qkv        7.29 us  4315 GB/s
    {SK_OP_GEMM, 6144, 2560, 2, {3, 10, 8, 32, 1, 192}},  // qkv        7.73 us  4073 GB/s
    {SK_OP_GEMM, 6144, 2560, 4, {3, 10, 8, 32, 1, 0}},  // qkv        7.84 us  4022 GB/s
    {SK_OP_GEMM, 6144, 2560, 8, {3, 10, 8, 32, 1, 192}},  // qkv        7.99 us  3955 GB/s
    {SK_OP_GEMM, 6144, 2560, 16, {3, 10, 8, 32, 1, 192}},  // qkv        8.43 us  3764 GB/s
    {SK_OP_PRE_GEMM, 6144, 2560, 8, {3, 10, 8, 16, 1, 192}},  // qkv consumer  9.07 us (32-row tiles 9.21)
    {SK_OP_PRE_GEMM, 6144, 2560, 16, {3, 10, 8, 16, 1, 0}},  // qkv consumer 10.13 us (32-row tiles 10.50)
    {SK_OP_PRE_GEMM, 6144, 2560, 64, {3, 10, 8, 16, 1, 64, 4}},  // consumer: 16-row groups (32-row consumers have 8 waves, too few for K)
    {SK_OP_PRE_GEMM, 6144, 2560, 128, {3, 10, 8, 16, 1, 32, 8}},  // consumer 24.0-26.3 us (eight 16-row groups; 30.2 at grid 64; two-operand wide path 31.3)
    {SK_OP_GEMM, 6144, 2560, 32, {3, 10, 8, 32, 1, 0}},  // qkv       10.22 us  3134 GB/s
    {SK_OP_GEMM, 6144, 2560, 40, {3, 10, 8, 16, 1, 0}},  // qkv       11.34 us  2835 GB/s (half ring)
    {SK_OP_GEMM, 6144, 2560, 48, {3, 10, 8, 16, 1, 128, 2}},  // qkv       11.33 us  2849 GB/s (two row groups; 12.0 half ring)
    {SK_OP_GEMM, 6144, 2560, 64, {3, 10, 8, 16, 1, 128, 2}},  // qkv       12.30 us  2558 GB/s (two row groups; 18.7 without)
    {SK_OP_GEMM, 6144, 2560, 128, {3, 10, 8, 16, 1, 64, 4}},  // qkv       16.6 us  (four row groups, one launch; 24.9 as two 64-row launches)
    {SK_OP_GEMM, 2560, 4096, 1, {2, 4, 2, 2, 1, 0}},  // o_proj     5.94 us  3531 GB/s
    // o_proj at M = 2-16: 12- or 10-row tiles, one per CU (214 or 256
    // workgroups of 16 waves; 16-row tiles leave 96 CUs idle): M = 8
    // 7.13 -> 6.86 us, M = 2 6.76 (GEMV) -> 6.68 us.
    {SK_OP_GEMM, 2560, 4096, 2, {3, 16, 8, 12, 1, 0}},  // o_proj     6.68 us  3144 GB/s
    {SK_OP_GEMM, 2560, 4096, 4, {3, 16, 8, 12, 1, 0}},  // o_proj     6.68 us  3145 GB/s
    {SK_OP_GEMM, 2560, 4096, 8, {3, 16, 8, 10, 1, 0}},  // o_proj     6.86 us  3066 GB/s
    {SK_OP_GEMM, 2560, 4096, 16, {3, 16, 8, 10, 1, 0}},  // o_proj     7.34 us  2870 GB/s
    {SK_OP_GEMM, 2560, 4096, 32, {3, 4, 32, 16, 1, 0}},  // o_proj     9.13 us  2343 GB/s
    {SK_OP_GEMM, 2560, 4096, 40, {3, 4, 32, 32, 1, 80, 3}},  // o_proj     9.96 us  2106 GB/s (three row groups; 11.6 without)
    {SK_OP_GEMM, 2560, 4096, 48, {3, 4, 32, 32, 1, 80, 3}},  // o_proj     9.92 us  2114 GB/s (three row groups; 11.5 without)
    {SK_OP_GEMM, 2560, 4096, 64, {3, 4, 32, 32, 1, 80, 3}},  // o_proj    12.37 us  1696 GB/s (three row groups; 14.8 without)
    {SK_OP_GEMM, 2560, 4096, 96, {3, 4, 32, 32, 1, 80, 3}},  // o_proj    12.7 us  (three 32-row groups; 14.8 with six)
    // 97-128 rows on the two-operand wide path (activation rows and weight
    // tile both staged in LDS, eight waves): 21.4 us against 22.1 for eight
    // row groups (24.9 as two 64-row launches).
    {SK_OP_GEMM, 2560, 4096, 128, {4, 8, 8, 32, 3, 0, 4}},  // o_proj    21.4 us
    {SK_OP_GATEUP, 9728, 2560, 1, {3, 10, 8, 16, 1, 203}},  // gate_up   17.31 us  5755 GB/s
    {SK_OP_RMSNORM_GATEUP, 9728, 2560, 1, {2, 4, 2, 2, 1, 0}},  // fused prologue beats 17.31 + a norm launch
    {SK_OP_GATEUP, 9728, 2560, 2, {3, 10, 8, 16, 1, 203}},  // gate_up   17.35 us  5746 GB/s
    {SK_OP_GATEUP, 9728, 2560, 4, {3, 10, 8, 16, 1, 203}},  // gate_up   17.37 us  5739 GB/s
    {SK_OP_GATEUP, 9728, 2560, 8, {3, 10, 8, 16, 1, 203}},  // gate_up   17.49 us  5707 GB/s
    {SK_OP_GATEUP, 9728, 2560, 16, {3, 10, 8, 16, 1, 203}},  // gate_up   18.13 us  5515 GB/s
    {SK_OP_GATEUP, 9728, 2560, 32, {3, 10, 8, 16, 1, 0}},  // gate_up   21.56 us  4656 GB/s (one partial buffer)
    {SK_OP_GATEUP, 9728, 2560, 40, {3, 10, 8, 16, 1, 0}},  // gate_up   24.79 us  4058 GB/s (half ring)
    {SK_OP_GATEUP, 9728, 2560, 48, {3, 10, 8, 16, 1, 128, 2}},  // gate_up   24.7 us  4080 GB/s (two row groups; 25.8 half ring)
    // 49-64 rows: the two-operand wide path (25.7 us against 26.5 for two ring
    // row groups in one run; 45.0 for one group)
    {SK_OP_GATEUP, 9728, 2560, 64, {4, 8, 8, 40, 1, 0, 4}},
    // 65-128 rows: the two-operand wide path, 40 + 40-row tiles (244
    // workgroups of eight waves): 36.1 us at 128 rows, 34.7 at 96, against
    // 42.9 and 38.1 for four row groups (55.9 as two 64-row launches).
    {SK_OP_GATEUP, 9728, 2560, 128, {4, 8, 8, 40, 1, 0, 4}},  // gate_up   36.1 us
    {SK_OP_PRE_GATEUP, 9728, 2560, 64, {3, 10, 8, 16, 1, 64, 4}},  // consumer, as for qkv
    // consumer at 65-128 rows: the two-operand wide path, 44.1 us at 128 rows
    // (eight 16-row ring groups 58.7-62.3; an add + RMSNorm launch and then
    // the plain projection 41.4: every workgroup normalises the whole
    // activation block while staging it, ~7 us of VALU work per launch)
    {SK_OP_PRE_GATEUP, 9728, 2560, 128, {4, 8, 8, 48, 1, 0, 4}},
    {SK_OP_GEMM, 2560, 9728, 1, {2, 2, 10, 2, 1, 0}},  // down      10.48 us  4754 GB/s
    // down at M = 3-8: eight waves of five 256-column chunks cover K = 9728
    // without a global split (13.1 -> 12.6 us at M = 8); at M = 2 the GEMV
    // of M = 1 is still ahead (11.33 us against 12.09).
    {SK_OP_GEMM, 2560, 9728, 2, {2, 2, 10, 2, 1, 0}},  // down      11.33 us  4398 GB/s
    {SK_OP_GEMM, 2560, 9728, 4, {3, 8, 40, 12, 1, 0}},  // down      12.16 us  4098 GB/s
    {SK_OP_GEMM, 2560, 9728, 8, {3, 8, 40, 12, 1, 0}},  // down      12.59 us  3962 GB/s
    // down at M = 9-16: 10-row tiles, one per CU, eight waves of five chunks
    // each (13.4 us against 14.0 for 32-row tiles in three K splits)
    {SK_OP_GEMM, 2560, 9728, 16, {3, 8, 40, 10, 1, 0}},  // down      13.4 us  3717 GB/s
    {SK_OP_GEMM, 2560, 9728, 32, {3, 4, 32, 32, 3, 0}},  // down      19.71 us  2568 GB/s
    {SK_OP_GEMM, 2560, 9728, 40, {3, 10, 8, 16, 4, 0}},  // down      19.62 us  2588 GB/s (half ring)
    {SK_OP_GEMM, 2560, 9728, 48, {4, 8, 8, 32, 3, 0, 4}},  // down      20.1 us (two-operand wide path; 20.6 half ring)
    // 49-64 rows: the two-operand wide path (20.2-20.6 us; the ring path
    // with five K splits 22.8-23.7)
    {SK_OP_GEMM, 2560, 9728, 64, {4, 8, 8, 32, 3, 0, 4}},  // down      20.58 us
    // 65-128 rows: the two-operand wide path, three K splits of 32-row tiles:
    // 34.4 us at 128 rows, 30.7 at 96 (four row groups with four splits 38.5
    // and 35.7; six splits of 64-row tiles within 0.4 us at twice the
    // partials).
    {SK_OP_GEMM, 2560, 9728, 128, {4, 8, 8, 32, 3, 0, 4}},  // down      34.4 us
    // Residual hand-off producers at decode row counts (the projection's
    // entries above use tile heights the hand-off cannot take).
    {SK_OP_RESID_GEMM, 2560, 4096, 8, {3, 16, 8, 16, 1, 0}},   // o_proj producer  7.46 us
    {SK_OP_RESID_GEMM, 2560, 4096, 16, {3, 4, 32, 16, 1, 0}},  // o_proj producer  7.91 us
    {SK_OP_RESID_GEMM, 2560, 9728, 8, {3, 8, 40, 16, 1, 0}},   // down producer   13.18 us (16.24 with three splits)
    // down producer at M = 9-16 (the decode step): 32-row tiles in three K
    // splits, 14.8 us (a producer tile holds whole 16-column groups, so the
    // plain plan's 10-row tiles do not apply)
    {SK_OP_RESID_GEMM, 2560, 9728, 16, {3, 13, 8, 32, 3, 240}},
    {SK_OP_RESID_GEMM, 2560, 9728, 64, {3, 10, 8, 16, 4, 128, 2}},  // down producer: its plain plan has no residual instance (64-row tiles)
    {SK_OP_LM_ARGMAX, 151936, 2560, 1, {3, 10, 8, 16, 1, 0}},  // lm_head  118.18 us  6583 GB/s
    {SK_OP_LM_ARGMAX, 151936, 2560, 2, {3, 10, 8, 32, 1, 0}},  // lm_head  117.50 us  6621 GB/s
    {SK_OP_LM_ARGMAX, 151936, 2560, 4, {3, 10, 8, 32, 1, 0}},  // lm_head  113.49 us  6855 GB/s
    {SK_OP_LM_ARGMAX, 151936, 2560, 8, {3, 10, 8, 32, 1, 0}},  // lm_head  113.31 us  6866 GB/s
    {SK_OP_LM_ARGMAX, 151936, 2560, 16, {3, 10, 8, 32, 1, 0}},  // lm_head  114.35 us  6804 GB/s
    {SK_OP_LM_ARGMAX, 151936, 2560, 32, {3, 5, 16, 16, 1, 0}},  // lm_head  119.79 us  6495 GB/s
    {SK_OP_LM_ARGMAX, 151936, 2560, 40, {3, 10, 8, 16, 1, 0}},  // lm_head  129.22 us  6022 GB/s (half ring)
    {SK_OP_LM_ARGMAX, 151936, 2560, 48, {3, 10, 8, 16, 1, 0}},  // lm_head  139.09 us  5594 GB/s (half ring)
    // 49-64 rows: the two-operand wide path over 128-row tiles (152-154 us;
    // two ring row groups 155-162, one 219)
    {SK_OP_LM_ARGMAX, 151936, 2560, 64, {4, 8, 8, 128, 1, 0, 4}},  // lm_head  153.8 us
    // lm_head + argmax at 65-128 rows: the two-operand wide path, every row
    // in one workgroup of eight waves over 128-row weight tiles (218 us at
    // 128 rows, 212 at 96; 96-row tiles 242 and 234, the weights-only-in-LDS
    // wide body 281 and 269, four row groups 306-309, two 64-row launches 362)
    {SK_OP_LM_ARGMAX, 151936, 2560, 128, {4, 8, 8, 128, 1, 0, 4}},
    {SK_OP_PRE_LM_ARGMAX, 151936, 2560, 64, {3, 10, 8, 16, 1, 64, 4}},  // consumer, as for qkv
    // consumer at 65-128 rows: the two-operand wide path, 238.7 us at 128 rows
    // (eight ring groups 412; the add + RMSNorm launch then the plain
    // projection 214.7)
    {SK_OP_PRE_LM_ARGMAX, 151936, 2560, 128, {4, 8, 8, 128, 1, 0, 4}},
    // lm_head logits at 33-64 rows: the two-operand wide path over 128-row
    // tiles (138-159 us; the ring plans of the fused argmax's entries store
    // logits at 139-185, two ring row groups 174-178)
    {SK_OP_GEMM, 151936, 2560, 40, {4, 8, 8, 128, 1, 0, 4}},
    {SK_OP_GEMM, 151936, 2560, 48, {4, 8, 8, 128, 1, 0, 4}},
    {SK_OP_GEMM, 151936, 2560, 64, {4, 8, 8, 128, 1, 0, 4}},
    // lm_head logits at 65-128 rows: as for the fused argmax, 209 us at 128
    // rows and 193 at 96 (96-row tiles 243 and 229, four row groups 304-342)
    {SK_OP_GEMM, 151936, 2560, 128, {4, 8, 8, 128, 1, 0, 4}},
};

// Tuned entry for op/N/K at the smallest tuned row count >= M among op's own
// entries and those of `also` (-1: none), op's own entry first at equal row
// counts.  The lm_head logits GEMM shares the fused argmax entries; a hand-off
// op shares its projection's.
const Tuned* tuned_lookup(int op, int M, int N, int K, int also = -1) {
  const Tuned* best = nullptr;
  for (const Tuned& t : kTuned) {
    const bool own = t.op == op;
    if (!(own || t.op == also) || t.N != N || t.K != K || t.M < M) continue;
    if (!best || t.M < best->M || (t.M == best->M && own)) best = &t;
  }
  return best;
}

// Heuristic for shapes outside the table: VALU GEMV for M <= 4 when K is a
// multiple of 512; otherwise the LDS-transposed MFMA path with one K chunk per
// wave and the fewest global splits that keep the waves within the compiled
// register budget; the register-fragment MFMA path as a last resort.
int heuristic_config(int op, int M, int N, int K, sk_config* out) {
  const bool gateup = (op == SK_OP_GATEUP);
  sk_config c;
  memset(&c, 0, sizeof(c));
  Plan pl;
  if (M <= 4 && op != SK_OP_LM_ARGMAX) {
    const int units = cdiv(K, 512);
    c.path = SK_PATH_GEMV;
    c.rows = 2;
    c.split = 1;
    c.waves = units < 4 ? units : 4;
    c.ku = cdiv(units, c.waves);
    if (plan_shape(op, M, N, K, c, &pl) == SK_OK && pl.lds <= kPrefLds) {
      *out = c;
      return SK_OK;
    }
  }
  const int MT = cdiv(M, 16);
  for (int ku : {16, 8}) {
    if (MT > 2 && ku == 16) continue;
    const int KW = 32 * ku;
    const int chunks = cdiv(K, KW);
    for (int split = 1; split <= 16; ++split) {
      if (op == SK_OP_LM_ARGMAX && split > 1) break;
      const int waves = cdiv(chunks, split);
      if (split > 1 && (split - 1) * waves >= chunks) break;
      c.path = SK_PATH_MFMA_LDS;
      c.rows = 16;
      c.split = split;
      c.waves = waves;
      c.ku = ku;
      if (plan_shape(op, M, N, K, c, &pl) == SK_OK && pl.lds <= kMaxLds) {
        *out = c;
        return SK_OK;
      }
    }
  }
  (void)gateup;
  return SK_ERR_SHAPE;
}

int mfma_search_config(int op, int M, int N, int K, int num_cu, sk_config* out) {
  (void)num_cu;   // the table is tuned for the MI355X's 256 CUs
  if (M < 1 || N < 1 || K < 32 || (K & 31) != 0) return SK_ERR_SHAPE;
  if (op != SK_OP_GEMM && op != SK_OP_GATEUP && op != SK_OP_LM_ARGMAX) return SK_ERR_CONFIG;
  const int Mk = M > kMaxM ? kMaxM : M;
  const int units = K / 32;
  const int MT = cdiv(Mk, 16);
  const bool gateup = (op == SK_OP_GATEUP);
  const int NT = gateup ? 2 : 1;
  // Prefer the largest K-unit bound (fewest waves sharing a tile, most bytes
  // in flight per wave) whose registers still allow the wave count, then the
  // fewest global K splits whose LDS fits the preferred budget.
  const int kus[] = {20, 16, 10, 8, 5};
  for (size_t pass = 0; pass < 2; ++pass) {
    const size_t lds_cap = pass == 0 ? kPrefLds : kMaxLds;
    for (int ku_cap : kus) {
      const int wmax = sk::max_waves_for_regs(sk::mfma_regs(MT, NT, ku_cap));
      if (sk::mfma_regs(MT, NT, ku_cap) > 256) continue;    // keep >= 2 waves per SIMD
      for (int split = 1; split <= 32; ++split) {
        if (op == SK_OP_LM_ARGMAX && split > 1) break;
        const int slice = cdiv(units, split);
        if (split > 1 && (split - 1) * slice >= units) break;
        const int waves = cdiv(slice, ku_cap);
        if (waves > wmax) continue;
        sk_config c;
        memset(&c, 0, sizeof(c));
        c.path = SK_PATH_MFMA;
        c.rows = 16;
        c.split = split;
        c.waves = waves;
        c.ku = cdiv(slice, waves);
        c.grid = 0;
        Plan pl;
        if (plan_shape(op, Mk, N, K, c, &pl) != SK_OK) continue;
        if (pl.lds > lds_cap) continue;
        *out = c;
        return SK_OK;
      }
    }
  }
  return SK_ERR_SHAPE;
}

int default_config(int op, int M, int N, int K, int num_cu, sk_config* out) {
  if (M < 1 || N < 1 || K < 32 || (K & 31) != 0) return SK_ERR_SHAPE;
  Plan pl;
  // Above kMaxM rows: a table entry that splits up to kMaxLaunchM rows into
  // row groups covers them in one launch; otherwise the call runs in kMaxM-row
  // chunks, each planned as below.
  if (M > kMaxM) {
    const int Ml = M < kMaxLaunchM ? M : kMaxLaunchM;
    const int bo = base_op(op);
    if (const Tuned* t = tuned_lookup(bo, Ml, N, K, bo == SK_OP_GEMM ? SK_OP_LM_ARGMAX : -1)) {
      if ((t->cfg.groups > 1 || t->cfg.path == SK_PATH_WIDE) && t->M > kMaxM &&
          plan_shape(op, Ml, N, K, t->cfg, &pl) == SK_OK) {
        *out = t->cfg;
        return SK_OK;
      }
    }
  }
  const int Mk = M > kMaxM ? kMaxM : M;
  // A norm op takes its own entry where the table has one (the fused GEMV
  // prologue can beat a faster projection plus a separate norm launch), else
  // its projection's configuration.
  if (is_norm_op(op)) {
    if (const Tuned* t = tuned_lookup(op, Mk, N, K)) {
      if (plan_shape(op, Mk, N, K, t->cfg, &pl) == SK_OK) {
        *out = t->cfg;
        return SK_OK;
      }
    }
  }
  op = base_op(op);
  if (!is_gemm_family(op)) return SK_ERR_CONFIG;
  if (const Tuned* t = tuned_lookup(op, Mk, N, K, op == SK_OP_GEMM ? SK_OP_LM_ARGMAX : -1)) {
    if (plan_shape(op, Mk, N, K, t->cfg, &pl) == SK_OK) {
      *out = t->cfg;
      return SK_OK;
    }
  }
  if (heuristic_config(op, Mk, N, K, out) == SK_OK) return SK_OK;
  return mfma_search_config(op, M, N, K, num_cu, out);
}

int resolve_config(int op, int M, int N, int K, const sk_config* cfg, sk_config* out) {
  if (cfg) {
    *out = *cfg;
    if (out->path == SK_PATH_AUTO) {
      sk_config d;
      int st = default_config(op, M, N, K, 0, &d);
      if (st) return st;
      *out = d;
    }
    return SK_OK;
  }
  return default_config(op, M, N, K, 0, out);
}

// Bind the kernel instance and compute the launch grid.
int bind_plan(Plan* pl, int num_cu, int* grid) {
  sk::KernelFn fn = plan_kernel(*pl);
  if (!fn) return SK_ERR_CONFIG;
  FnInfo fi;
  int st = fn_info(reinterpret_cast<const void*>(fn), &fi);
  if (st) return st;
  const int threads = 64 * pl->cfg.waves;
  if (threads > fi.max_threads) return SK_ERR_CONFIG;
  pl->fn = fn;
  const int S = pl->cfg.split;
  if (pl->cfg.grid > 0) {
    *grid = pl->cfg.grid;
  } else {
    // Resident workgroups per K split from the occupancy at one staged tile,
    // then as many tiles per workgroup as that needs (evened out so the last
    // round is not a partial one), shrunk while the staging exceeds the
    // preferred LDS budget.
    const int per_cu = occupancy(reinterpret_cast<const void*>(fn), threads, pl->lds);
    long cap = (long)per_cu * num_cu / S;
    if (cap < 1) cap = 1;
    int per_split = pl->nrb < cap ? pl->nrb : (int)cap;
    if (per_split > kMaxGrid) per_split = kMaxGrid;
    int tiles_per = cdiv(pl->nrb, per_split);
    if (epi_base(pl->epi) != sk::EPI_ARGMAX) {
      // Never below the tiles per workgroup that keep the grid within
      // kMaxGrid (lm_head logits: 9496 tiles); past the preferred budget the
      // staging may use the whole LDS.
      const int min_tiles = cdiv(pl->nrb, kMaxGrid);
      const size_t budget = pl->pre_lds + pl->parts_lds + (size_t)min_tiles * pl->stage_elem > kPrefLds ? kMaxLds
                                                                                                      : kPrefLds;
      while (tiles_per > min_tiles && plan_lds(*pl, 0, tiles_per) > budget) --tiles_per;
    }
    per_split = cdiv(pl->nrb, tiles_per);
    if (per_split > kMaxGrid) return SK_ERR_CONFIG;
    *grid = per_split * S;
  }
  const int tiles_per = cdiv(pl->nrb, *grid / S);
  pl->lds = epi_base(pl->epi) == sk::EPI_ARGMAX ? pl->lds : plan_lds(*pl, 0, tiles_per);
  if (pl->lds > kMaxLds) return SK_ERR_CONFIG;
  if (pl->lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)pl->lds) != hipSuccess)
    return SK_ERR_CONFIG;
  return SK_OK;
}

// Device address of the current device's copy of `scratch`, looked up once
// per device with that device current (each GPU holds its own copy at its own
// address).
void* g_scratch_ptr[64];
int g_scratch_status[64] = {};   // 0: not looked up yet, else sk_status + 1

int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return SK_ERR_DEVICE;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_scratch_status[dev] == 0) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = p;
    g_scratch_status[dev] = (e == hipSuccess && p) ? SK_OK + 1 : SK_ERR_DEVICE + 1;
  }
  *out = g_scratch_ptr[dev];
  return g_scratch_status[dev] - 1;
}

bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + bbytes && pb < pa + abytes;
}

int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SK_OK : SK_ERR_LAUNCH;
}

// Residual add + RMSNorm prologue inputs of the norm ops (x is the A operand).
struct NormIn {
  const sk_bf16* y;
  const sk_bf16* w;
  float eps;
  sk_bf16* xout;
};

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Plans of one call: rows beyond one launch's (launch_rows) are processed in
// chunks of that many rows (each streaming the weights once more), so a call
// has at most two distinct chunk sizes.  Also the workspace it needs: the
// plans' counters and partials, then, when the norm prologue runs as its own
// launch, the normalised activations [M, K] at offset `norm_off`.
struct CallPlan {
  Plan plans[2];
  int chunk = 0;                // rows per launch
  int chunk_rows[2] = {0, 0};
  int nplans = 0;
  size_t base_need = 0;
  size_t norm_off = 0;
  size_t need = 0;
  bool fused = false;
};

// Rows one launch of a call covers: up to kMaxLaunchM when the configuration
// for that many rows splits them into row groups, else kMaxM.
int launch_rows(int op, int M, int N, int K, const sk_config* cfg) {
  if (M <= kMaxM) return kMaxM;
  const int R = M < kMaxLaunchM ? M : kMaxLaunchM;
  sk_config c;
  Plan pl;
  if (resolve_config(op, R, N, K, cfg, &c) == SK_OK && (c.groups > 1 || c.path == SK_PATH_WIDE) &&
      plan_shape(op, R, N, K, c, &pl) == SK_OK)
    return kMaxLaunchM;
  return kMaxM;
}

int plan_call(int op, int M, int N, int K, const sk_config* cfg, CallPlan* cp) {
  const int chunk = launch_rows(op, M, N, K, cfg);
  cp->chunk = chunk;
  cp->chunk_rows[0] = M < chunk ? M : chunk;
  cp->chunk_rows[1] = M % chunk;
  cp->nplans = (M > chunk && (M % chunk) != 0) ? 2 : 1;
  for (int i = 0; i < cp->nplans; ++i) {
    sk_config c;
    int st = resolve_config(op, cp->chunk_rows[i], N, K, cfg, &c);
    if (st) return st;
    // A configuration with row groups applies to every launch of the call; a
    // launch with too few rows to give each group one (the remainder after
    // 128-row launches, e.g. one row of 129) runs with as many groups as
    // hold a row, so the configuration default_config returns for the whole
    // call is accepted for every launch.
    if (cp->nplans == 2 && i == 1 && c.groups > 1 && c.path != SK_PATH_WIDE) {
      const int rows = cp->chunk_rows[i];
      int g = c.groups;
      while (g > 1 && (g - 1) * cdiv(rows, g) >= rows) --g;
      c.groups = g > 1 ? g : 0;
    }
    st = plan_shape(op, cp->chunk_rows[i], N, K, c, &cp->plans[i]);
    if (st) return st;
  }
  cp->fused = is_norm_op(op) && cp->plans[0].fused && (cp->nplans == 1 || cp->plans[1].fused);
  if (is_norm_op(op) && !cp->fused) {   // every chunk then takes the separate prologue
    for (int i = 0; i < cp->nplans; ++i) {
      const sk_config c = cp->plans[i].cfg;
      int st = plan_shape_impl(base_op(op), cp->chunk_rows[i], N, K, c, false, &cp->plans[i]);
      if (st) return st;
      cp->plans[i].norm = true;
    }
  }
  cp->base_need = 0;
  for (int i = 0; i < cp->nplans; ++i) {
    const size_t n = plan_workspace(op, cp->chunk_rows[i], N, cp->plans[i]);
    if (n > cp->base_need) cp->base_need = n;
  }
  cp->need = cp->base_need;
  if (is_norm_op(op) && !cp->fused) {
    cp->norm_off = align256(cp->base_need);
    cp->need = cp->norm_off + (size_t)M * K * sizeof(sk_bf16);
  }
  return SK_OK;
}

// Shared driver of the GEMM-family ops.  nrm != nullptr: A is x and the
// projection consumes rmsnorm(x + y) (op is then a SK_OP_RMSNORM_* op).
int run_gemm_family(int op, const sk_bf16* A, int64_t lda, const NormIn* nrm, const sk_bf16* W0, const sk_bf16* W1,
                    int64_t ldw, sk_bf16* C, int64_t ldc, int64_t* ids, float* maxv, int M, int N, int K,
                    const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream,
                    bool noalloc = false) {
  const int bop = base_op(op);
  if (M < 0 || N < 1 || K < 32) return SK_ERR_SHAPE;
  if (M == 0) return SK_OK;   // empty batch: nothing to read or write (pointers may be NULL)
  if (!A || !W0 || (bop == SK_OP_GATEUP && !W1)) return SK_ERR_NULL;
  if (bop == SK_OP_LM_ARGMAX ? (!ids || !maxv) : !C) return SK_ERR_NULL;
  if (nrm && (!nrm->y || !nrm->w || !nrm->xout)) return SK_ERR_NULL;
  if ((K & 31) != 0 || lda < K || ldw < K || (bop != SK_OP_LM_ARGMAX && ldc < N)) return SK_ERR_SHAPE;
  if (nrm && K > sk::RMS_THREADS * 8 * sk::RMS_MAX_CHUNKS) return SK_ERR_SHAPE;
  if (!aligned16(A) || !aligned16(W0) || (W1 && !aligned16(W1)) || (lda & 7) || (ldw & 7)) return SK_ERR_ALIGN;
  if (nrm && (!aligned16(nrm->y) || !aligned16(nrm->w) || !aligned16(nrm->xout))) return SK_ERR_ALIGN;
  // Outputs are written while other workgroups may still read the inputs.
  const size_t a_bytes = ((size_t)(M - 1) * lda + K) * sizeof(sk_bf16);
  const size_t c_bytes = bop == SK_OP_LM_ARGMAX ? 0 : ((size_t)(M - 1) * ldc + N) * sizeof(sk_bf16);
  if (c_bytes && overlaps(C, c_bytes, A, a_bytes)) return SK_ERR_ALIAS;
  if (nrm) {
    if (overlaps(nrm->xout, a_bytes, A, a_bytes) || overlaps(nrm->xout, a_bytes, nrm->y, a_bytes))
      return SK_ERR_ALIAS;
    if (c_bytes && (overlaps(C, c_bytes, nrm->y, a_bytes) || overlaps(C, c_bytes, nrm->xout, a_bytes)))
      return SK_ERR_ALIAS;
  }
  // Validate every chunk's plan and the workspace before enqueuing anything.
  CallPlan cp;
  int st = plan_call(op, M, N, K, cfg, &cp);
  if (st) return st;
  if (noalloc) {   // the library's static scratch stands in for the workspace
    if (cp.need > SK_NOALLOC_SCRATCH_BYTES) return SK_ERR_SCRATCH;
  } else if (cp.need > 0 && (!ws || ws_bytes < cp.need)) {
    return SK_ERR_WORKSPACE;
  }
  int num_cu = 0;
  st = device_info(&num_cu);
  if (st) return st;
  int grids[2];
  for (int i = 0; i < cp.nplans; ++i) {
    st = bind_plan(&cp.plans[i], num_cu, &grids[i]);
    if (st) return st;
  }
  if (noalloc && cp.need > 0) {
    if ((st = scratch_address(&ws))) return st;
    ws_bytes = SK_NOALLOC_SCRATCH_BYTES;
    // The arrival counters must start at zero.  Every finished call leaves
    // them at zero, but the array keeps whatever the last call on this GPU
    // left, so the counters this call uses are cleared first (a fill kernel,
    // which also replays correctly from a captured graph).
    size_t tb = 0;
    for (int i = 0; i < cp.nplans; ++i) {
      const size_t t = plan_tickets(bop, cp.plans[i]);
      tb = t > tb ? t : tb;
    }
    sk::clear_words_kernel<<<dim3(1), dim3(256), 0, stream>>>(static_cast<unsigned*>(ws), (int)(tb / 4));
    if ((st = launch_status())) return st;
  }
  // Separate prologue: xout and the normalised rows (in the workspace) first.
  const sk_bf16* Ause = A;
  int64_t ldause = lda;
  if (nrm && !cp.fused) {
    sk_bf16* nb = reinterpret_cast<sk_bf16*>(static_cast<char*>(ws) + cp.norm_off);
    sk::add_rmsnorm_kernel<<<dim3(M), dim3(sk::RMS_THREADS), 0, stream>>>(A, nrm->y, nrm->w, nrm->eps, nrm->xout, nb,
                                                                         K, lda, K);
    if ((st = launch_status())) return st;
    Ause = nb;
    ldause = K;
  }
  for (int m0 = 0; m0 < M; m0 += cp.chunk) {
    const int rows = (M - m0) < cp.chunk ? (M - m0) : cp.chunk;
    const int pi = rows == cp.chunk_rows[0] ? 0 : 1;
    const Plan& pl = cp.plans[pi];
    const int grid = grids[pi];
    sk::Args a;
    memset(&a, 0, sizeof(a));
    a.A = Ause + (int64_t)m0 * ldause;
    a.W0 = W0;
    a.W1 = W1;
    a.C = C ? C + (int64_t)m0 * ldc : nullptr;
    if (ws) {
      const size_t tb = plan_tickets(bop, pl);
      a.tickets = static_cast<unsigned*>(ws);
      a.part = reinterpret_cast<float*>(static_cast<char*>(ws) + tb);
      a.best = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + tb);
    }
    if (bop == SK_OP_LM_ARGMAX) {   // the fused argmax finishes into ids / maxv
      a.C = reinterpret_cast<sk_bf16*>(ids + m0);
      a.part = maxv + m0;
    }
    if (nrm && cp.fused) {
      a.Y = nrm->y + (int64_t)m0 * lda;
      a.NW = nrm->w;
      a.XO = nrm->xout + (int64_t)m0 * lda;
      a.eps = nrm->eps;
    }
    a.lda = ldause;
    a.ldw = ldw;
    a.ldc = ldc;
    a.M = rows;
    a.N = N;
    a.K = K;
    a.S = pl.cfg.split;
    a.slice_units = pl.slice_units;
    a.ku = pl.cfg.ku;
    a.nrb = pl.nrb;
    a.tr = pl.tr;
    a.nw = pl.cfg.waves;
    a.grid = grid;
    a.rbstep = grid / pl.cfg.split;
    a.pbuf = pl.pbuf;
    a.groups = pl.groups;
    a.mrows = pl.mrows;
    pl.fn<<<dim3(grid * pl.groups), dim3(64 * pl.cfg.waves), pl.lds, stream>>>(a);
    if ((st = launch_status())) return st;
  }
  return SK_OK;
}

// ---------------------------------------------------------------------------
// Residual hand-off ops (SK_OP_RESID_GEMM, SK_OP_PRE_*).
// ---------------------------------------------------------------------------
bool is_handoff_op(int op) { return op >= SK_OP_RESID_GEMM && op <= SK_OP_PRE_LM_ARGMAX; }
int handoff_base(int op) {
  return op == SK_OP_PRE_GATEUP ? SK_OP_GATEUP : (op == SK_OP_PRE_LM_ARGMAX ? SK_OP_LM_ARGMAX : SK_OP_GEMM);
}
int handoff_variant(int op) { return op == SK_OP_RESID_GEMM ? 2 : 1; }

// Configuration of a hand-off op: the explicit one, else the projection's
// tuned one when it is a supported ring configuration, else a ring one with
// one 256-column chunk per wave (four for a producer whose K needs more than
// 16 waves), one K split.
int handoff_config(int op, int M, int N, int K, const sk_config* cfg, sk_config* out) {
  const int bop = handoff_base(op), variant = handoff_variant(op);
  Plan pl;
  if (cfg && cfg->path != SK_PATH_AUTO) {
    *out = *cfg;
    return SK_OK;
  }
  // The table entry of the hand-off op or of its projection at the nearest
  // row count (the hand-off op's own first), then the projection's default.
  if (const Tuned* t = tuned_lookup(op, M, N, K, bop)) {
    if (plan_shape_impl(bop, M, N, K, t->cfg, false, &pl, variant) == SK_OK) {
      *out = t->cfg;
      return SK_OK;
    }
  }
  sk_config d;
  if (default_config(bop, M, N, K, 0, &d) == SK_OK && plan_shape_impl(bop, M, N, K, d, false, &pl, variant) == SK_OK) {
    *out = d;
    return SK_OK;
  }
  // Ring candidates in order: one K split with 256-column chunks, then (the
  // producer only) four chunks per wave, then global K splits.  The hand-off
  // instances hold at most 32 rows (consumers: 16, and 4 per wave), so more
  // rows run as row groups, each with a grid of one workgroup per tile and
  // split, rounded up to a multiple of 8 split-sized runs.
  for (int ku : {8, 32}) {
    if (ku == 32 && variant == 1) continue;
    for (int split = 1; split <= (variant == 2 ? 4 : 1); ++split) {
      memset(&d, 0, sizeof(d));
      d.path = SK_PATH_MFMA_LDS;
      d.rows = 16;
      d.ku = ku;
      d.split = split;
      const int units = (K + 32 * ku - 1) / (32 * ku);
      d.waves = (units + split - 1) / split;
      const int group_rows = variant == 1 ? (4 * d.waves < 16 ? 4 * d.waves : 16) : 32;
      if (M > group_rows) {
        d.groups = cdiv(M, group_rows);
        d.grid = cdiv(cdiv(N, 16) * split, 8 * split) * 8 * split;
      }
      if (d.waves <= 16 && plan_shape_impl(bop, M, N, K, d, false, &pl, variant) == SK_OK) {
        *out = d;
        return SK_OK;
      }
    }
  }
  return SK_ERR_CONFIG;
}

int plan_handoff(int op, int M, int N, int K, const sk_config* cfg, Plan* pl) {
  if (M < 1 || M > kMaxLaunchM || N < 1 || K < 32) return SK_ERR_SHAPE;
  sk_config c;
  int st = handoff_config(op, M, N, K, cfg, &c);
  if (st) return st;
  return plan_shape_impl(handoff_base(op), M, N, K, c, false, pl, handoff_variant(op));
}

size_t handoff_workspace(int op, int M, int N, int K, const sk_config* cfg) {
  Plan pl;
  if (plan_handoff(op, M, N, K, cfg, &pl)) return 0;
  return plan_workspace(handoff_base(op), M, N, pl);
}

struct Handoff {
  const sk_bf16* r;     // producer: residual in
  sk_bf16* r_out;       // producer: residual out
  int64_t ldr;
  float* sq;            // producer: partial sums out / consumer: in
  const sk_bf16* w;     // consumer: norm weights
  float eps;
};

int run_handoff(int op, const sk_bf16* A, int64_t lda, const Handoff& h, const sk_bf16* W0, const sk_bf16* W1,
                int64_t ldw, sk_bf16* C, int64_t ldc, int64_t* ids, float* maxv, int M, int N, int K,
                const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream) {
  const int bop = handoff_base(op);
  const bool resid = handoff_variant(op) == 2;
  if (M < 0 || N < 1 || K < 32 || M > kMaxLaunchM) return SK_ERR_SHAPE;
  if (M == 0) return SK_OK;
  if (!A || !W0 || (bop == SK_OP_GATEUP && !W1) || !h.sq) return SK_ERR_NULL;
  if (resid ? (!h.r || !h.r_out) : !h.w) return SK_ERR_NULL;
  if (!resid && (bop == SK_OP_LM_ARGMAX ? (!ids || !maxv) : !C)) return SK_ERR_NULL;
  if ((K & 31) != 0 || lda < K || ldw < K) return SK_ERR_SHAPE;
  if (!resid && bop != SK_OP_LM_ARGMAX && ldc < N) return SK_ERR_SHAPE;
  if (resid && h.ldr < N) return SK_ERR_SHAPE;
  if (!aligned16(A) || !aligned16(W0) || (W1 && !aligned16(W1)) || (lda & 7) || (ldw & 7)) return SK_ERR_ALIGN;
  if (!resid && (!aligned16(h.w) || (reinterpret_cast<uintptr_t>(h.sq) & 3))) return SK_ERR_ALIGN;
  if (resid && ((reinterpret_cast<uintptr_t>(h.r) | reinterpret_cast<uintptr_t>(h.r_out)) & 1)) return SK_ERR_ALIGN;
  const int sq_ld = resid ? (N + 15) / 16 : K / 16;
  const size_t a_bytes = ((size_t)(M - 1) * lda + K) * sizeof(sk_bf16);
  const size_t sq_bytes = (size_t)M * sq_ld * sizeof(float);
  if (resid) {
    const size_t r_bytes = ((size_t)(M - 1) * h.ldr + N) * sizeof(sk_bf16);
    // r_out may equal r (each element is read and written by one thread), but
    // no output may overlap the projection's input or the other output.
    if (overlaps(h.r_out, r_bytes, A, a_bytes) || overlaps(h.sq, sq_bytes, A, a_bytes) ||
        overlaps(h.sq, sq_bytes, h.r_out, r_bytes) || overlaps(h.sq, sq_bytes, h.r, r_bytes))
      return SK_ERR_ALIAS;
    if (h.r != h.r_out && overlaps(h.r_out, r_bytes, h.r, r_bytes)) return SK_ERR_ALIAS;
  } else if (bop != SK_OP_LM_ARGMAX) {
    const size_t c_bytes = ((size_t)(M - 1) * ldc + N) * sizeof(sk_bf16);
    if (overlaps(C, c_bytes, A, a_bytes) || overlaps(C, c_bytes, h.sq, sq_bytes)) return SK_ERR_ALIAS;
  }
  Plan pl;
  int st = plan_handoff(op, M, N, K, cfg, &pl);
  if (st) return st;
  const size_t need = plan_workspace(bop, M, N, pl);
  if (need > 0 && (!ws || ws_bytes < need)) return SK_ERR_WORKSPACE;
  int num_cu = 0;
  if ((st = device_info(&num_cu))) return st;
  int grid = 0;
  if ((st = bind_plan(&pl, num_cu, &grid))) return st;
  sk::Args a;
  memset(&a, 0, sizeof(a));
  a.A = A;
  a.W0 = W0;
  a.W1 = W1;
  a.C = C;
  if (ws) {
    const size_t tb = plan_tickets(bop, pl);
    a.tickets = static_cast<unsigned*>(ws);
    a.part = reinterpret_cast<float*>(static_cast<char*>(ws) + tb);
    a.best = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + tb);
  }
  if (bop == SK_OP_LM_ARGMAX) {
    a.C = reinterpret_cast<sk_bf16*>(ids);
    a.part = maxv;
  }
  a.R = h.r;
  a.RO = h.r_out;
  a.ldr = h.ldr;
  a.SQ = h.sq;
  a.sq_ld = sq_ld;
  a.NW = h.w;
  a.eps = h.eps;
  a.lda = lda;
  a.ldw = ldw;
  a.ldc = ldc;
  a.M = M;
  a.N = N;
  a.K = K;
  a.S = pl.cfg.split;
  a.slice_units = pl.slice_units;
  a.ku = pl.cfg.ku;
  a.nrb = pl.nrb;
  a.tr = pl.tr;
  a.nw = pl.cfg.waves;
  a.grid = grid;
  a.rbstep = grid / pl.cfg.split;
  a.pbuf = pl.pbuf;
  a.groups = pl.groups;
  a.mrows = pl.mrows;
  pl.fn<<<dim3(grid * pl.groups), dim3(64 * pl.cfg.waves), pl.lds, stream>>>(a);
  return launch_status();
}

}  // namespace

extern "C" {

int sk_version(void) { return (0 << 16) | 3; }

const char* sk_strerror(int status) {
  switch (status) {
    case SK_OK: return "ok";
    case SK_ERR_NULL: return "a required pointer is NULL";
    case SK_ERR_SHAPE: return "shape or stride out of the supported range";
    case SK_ERR_ALIGN: return "pointer or stride not aligned for 16-byte loads";
    case SK_ERR_WORKSPACE: return "workspace missing or too small";
    case SK_ERR_CONFIG: return "launch configuration invalid for this shape";
    case SK_ERR_LAUNCH: return "kernel launch failed";
    case SK_ERR_DEVICE: return "no usable gfx950 device";
    case SK_ERR_ALIAS: return "output overlaps an input";
    case SK_ERR_SCRATCH: return "call needs more than the library's static scratch (SK_NOALLOC_SCRATCH_BYTES)";
  }
  return "unknown status";
}

int sk_default_config(int op, int M, int N, int K, int num_cu, sk_config* out) {
  if (!out) return SK_ERR_NULL;
  if (is_handoff_op(op)) return handoff_config(op, M > kMaxLaunchM ? kMaxLaunchM : M, N, K, nullptr, out);
  if (!is_gemm_family(base_op(op))) return SK_ERR_CONFIG;
  return default_config(op, M, N, K, num_cu, out);
}

int sk_check_config(int op, int M, int N, int K, const sk_config* cfg) {
  if (!cfg) return SK_ERR_NULL;
  if (is_handoff_op(op)) {
    Plan pl;
    return plan_handoff(op, M, N, K, cfg, &pl);
  }
  if (M < 1) return SK_ERR_SHAPE;
  // Every launch of the call (a row count past one launch's takes several,
  // the last one shorter) must accept the configuration.
  CallPlan cp;
  return plan_call(op, M, N, K, cfg, &cp);
}

size_t sk_workspace_bytes(int op, int M, int N, int K, const sk_config* cfg) {
  if (is_handoff_op(op)) return M < 1 ? 0 : handoff_workspace(op, M, N, K, cfg);
  if (op == SK_OP_ARGMAX) {
    if (M < 1 || N < 1) return 0;
    return ticket_bytes(1) + (size_t)M * sizeof(unsigned long long);
  }
  if (M < 1 || !is_gemm_family(base_op(op))) return 0;
  CallPlan cp;
  if (plan_call(op, M, N, K, cfg, &cp)) return 0;
  return cp.need;
}

int sk_gemm_bf16(const sk_bf16* A, int64_t lda, const sk_bf16* W, int64_t ldw, sk_bf16* C, int64_t ldc, int M, int N,
                 int K, const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream) {
  return run_gemm_family(SK_OP_GEMM, A, lda, nullptr, W, nullptr, ldw, C, ldc, nullptr, nullptr, M, N, K, cfg, ws,
                         ws_bytes, stream);
}

int sk_gemm_bf16_noalloc(const sk_bf16* A, int64_t lda, const sk_bf16* W, int64_t ldw, sk_bf16* C, int64_t ldc,
                         int M, int N, int K, const sk_config* cfg, hipStream_t stream) {
  return run_gemm_family(SK_OP_GEMM, A, lda, nullptr, W, nullptr, ldw, C, ldc, nullptr, nullptr, M, N, K, cfg, nullptr,
                         0, stream, /*noalloc=*/true);
}

int sk_gateup_swiglu_bf16(const sk_bf16* A, int64_t lda, const sk_bf16* Wg, const sk_bf16* Wu, int64_t ldw,
                          sk_bf16* Out, int64_t ldo, int M, int I, int K, const sk_config* cfg, void* ws,
                          size_t ws_bytes, hipStream_t stream) {
  return run_gemm_family(SK_OP_GATEUP, A, lda, nullptr, Wg, Wu, ldw, Out, ldo, nullptr, nullptr, M, I, K, cfg, ws,
                         ws_bytes, stream);
}

int sk_lm_argmax_bf16(const sk_bf16* A, int64_t lda, const sk_bf16* W, int64_t ldw, int64_t* ids, float* maxv, int M,
                      int V, int K, const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream) {
  return run_gemm_family(SK_OP_LM_ARGMAX, A, lda, nullptr, W, nullptr, ldw, nullptr, 0, ids, maxv, M, V, K, cfg, ws,
                         ws_bytes, stream);
}

int sk_rmsnorm_gemm_bf16(const sk_bf16* x, const sk_bf16* y, const sk_bf16* w_norm, float eps, sk_bf16* xout,
                         int64_t ldx, const sk_bf16* W, int64_t ldw, sk_bf16* C, int64_t ldc, int M, int N, int K,
                         const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream) {
  const NormIn n{y, w_norm, eps, xout};
  return run_gemm_family(SK_OP_RMSNORM_GEMM, x, ldx, &n, W, nullptr, ldw, C, ldc, nullptr, nullptr, M, N, K, cfg, ws,
                         ws_bytes, stream);
}

int sk_rmsnorm_gateup_swiglu_bf16(const sk_bf16* x, const sk_bf16* y, const sk_bf16* w_norm, float eps,
                                  sk_bf16* xout, int64_t ldx, const sk_bf16* Wg, const sk_bf16* Wu, int64_t ldw,
                                  sk_bf16* Out, int64_t ldo, int M, int I, int K, const sk_config* cfg, void* ws,
                                  size_t ws_bytes, hipStream_t stream) {
  const NormIn n{y, w_norm, eps, xout};
  return run_gemm_family(SK_OP_RMSNORM_GATEUP, x, ldx, &n, Wg, Wu, ldw, Out, ldo, nullptr, nullptr, M, I, K, cfg, ws,
                         ws_bytes, stream);
}

int sk_rmsnorm_lm_argmax_bf16(const sk_bf16* x, const sk_bf16* y, const sk_bf16* w_norm, float eps, sk_bf16* xout,
                              int64_t ldx, const sk_bf16* W, int64_t ldw, int64_t* ids, float* maxv, int M, int V,
                              int K, const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream) {
  const NormIn n{y, w_norm, eps, xout};
  return run_gemm_family(SK_OP_RMSNORM_LM_ARGMAX, x, ldx, &n, W, nullptr, ldw, nullptr, 0, ids, maxv, M, V, K, cfg, ws,
                         ws_bytes, stream);
}

int sk_argmax_bf16(const sk_bf16* L, int64_t ld, int M, int V, int64_t* ids, float* maxv, void* ws, size_t ws_bytes,
                   hipStream_t stream) {
  if (M < 0 || V < 1 || ld < V) return SK_ERR_SHAPE;
  if (M == 0) return SK_OK;
  if (!L || !ids || !maxv) return SK_ERR_NULL;
  if (M > 65535) return SK_ERR_SHAPE;
  const int chunks = cdiv(V, kArgmaxChunk);
  const size_t need = ticket_bytes(1) + (size_t)M * sizeof(unsigned long long);
  if (!ws || ws_bytes < need) return SK_ERR_WORKSPACE;
  int num_cu = 0;
  int st = device_info(&num_cu);
  if (st) return st;
  unsigned* ticket = static_cast<unsigned*>(ws);
  unsigned long long* best = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + ticket_bytes(1));
  const int vec = (aligned16(L) && (ld & 7) == 0) ? 1 : 0;
  sk::argmax_kernel<<<dim3(chunks, M), dim3(sk::ARGMAX_THREADS), 0, stream>>>(L, ld, M, V, kArgmaxChunk, vec, best,
                                                                             ticket, ids, maxv);
  return launch_status();
}

int sk_add_rmsnorm_bf16(const sk_bf16* x, const sk_bf16* y, const sk_bf16* w, float eps, sk_bf16* xout, sk_bf16* out,
                        int M, int K, int64_t ld, hipStream_t stream) {
  if (M < 0 || K < 8 || (K & 7) || K > sk::RMS_THREADS * 8 * sk::RMS_MAX_CHUNKS || ld < K) return SK_ERR_SHAPE;
  if (M == 0) return SK_OK;
  if (!x || !y || !w || !xout || !out) return SK_ERR_NULL;
  if (!aligned16(x) || !aligned16(y) || !aligned16(w) || !aligned16(xout) || !aligned16(out) || (ld & 7))
    return SK_ERR_ALIGN;
  if (M > 65535) return SK_ERR_SHAPE;
  // xout may be x or y itself (each element is read before the same thread
  // writes it), but must not partially overlap them; out overlaps nothing.
  const size_t bytes = ((size_t)(M - 1) * ld + K) * sizeof(sk_bf16);
  if ((xout != x && overlaps(xout, bytes, x, bytes)) || (xout != y && overlaps(xout, bytes, y, bytes)) ||
      overlaps(out, bytes, x, bytes) || overlaps(out, bytes, y, bytes) || overlaps(out, bytes, xout, bytes))
    return SK_ERR_ALIAS;
  int num_cu = 0;
  int st = device_info(&num_cu);
  if (st) return st;
  sk::add_rmsnorm_kernel<<<dim3(M), dim3(sk::RMS_THREADS), 0, stream>>>(x, y, w, eps, xout, out, K, ld, ld);
  return launch_status();
}

int sk_swiglu_bf16(const sk_bf16* gu, int64_t ld_gu, sk_bf16* out, int64_t ld_out, int M, int I, hipStream_t stream) {
  if (M < 0 || I < 1 || ld_gu < 2 * (int64_t)I || ld_out < I) return SK_ERR_SHAPE;
  if (M == 0) return SK_OK;
  if (!gu || !out) return SK_ERR_NULL;
  const size_t in_bytes = ((size_t)(M - 1) * ld_gu + 2 * (size_t)I) * sizeof(sk_bf16);
  const size_t out_bytes = ((size_t)(M - 1) * ld_out + I) * sizeof(sk_bf16);
  if (overlaps(out, out_bytes, gu, in_bytes)) return SK_ERR_ALIAS;
  int num_cu = 0;
  int st = device_info(&num_cu);
  if (st) return st;
  const long total = (long)M * I;
  long g = (total + 255) / 256;
  if (g > 8L * num_cu * 8) g = 8L * num_cu * 8;
  sk::swiglu_kernel<<<dim3((unsigned)g), dim3(256), 0, stream>>>(gu, ld_gu, out, ld_out, M, I);
  return launch_status();
}


int sk_gemm_residual_bf16(const sk_bf16* A, int64_t lda, const sk_bf16* W, int64_t ldw, const sk_bf16* r,
                          sk_bf16* r_out, int64_t ldr, float* sq, int M, int N, int K, const sk_config* cfg, void* ws,
                          size_t ws_bytes, hipStream_t stream) {
  Handoff h{r, r_out, ldr, sq, nullptr, 0.f};
  return run_handoff(SK_OP_RESID_GEMM, A, lda, h, W, nullptr, ldw, nullptr, 0, nullptr, nullptr, M, N, K, cfg, ws,
                     ws_bytes, stream);
}

int sk_rmsnorm_pre_gemm_bf16(const sk_bf16* x, int64_t ldx, const float* sq, const sk_bf16* w_norm, float eps,
                             const sk_bf16* W, int64_t ldw, sk_bf16* C, int64_t ldc, int M, int N, int K,
                             const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream) {
  Handoff h{nullptr, nullptr, 0, const_cast<float*>(sq), w_norm, eps};
  return run_handoff(SK_OP_PRE_GEMM, x, ldx, h, W, nullptr, ldw, C, ldc, nullptr, nullptr, M, N, K, cfg, ws, ws_bytes,
                     stream);
}

int sk_rmsnorm_pre_gateup_swiglu_bf16(const sk_bf16* x, int64_t ldx, const float* sq, const sk_bf16* w_norm,
                                      float eps, const sk_bf16* Wg, const sk_bf16* Wu, int64_t ldw, sk_bf16* Out,
                                      int64_t ldo, int M, int I, int K, const sk_config* cfg, void* ws,
                                      size_t ws_bytes, hipStream_t stream) {
  Handoff h{nullptr, nullptr, 0, const_cast<float*>(sq), w_norm, eps};
  return run_handoff(SK_OP_PRE_GATEUP, x, ldx, h, Wg, Wu, ldw, Out, ldo, nullptr, nullptr, M, I, K, cfg, ws,
                     ws_bytes, stream);
}

int sk_rmsnorm_pre_lm_argmax_bf16(const sk_bf16* x, int64_t ldx, const float* sq, const sk_bf16* w_norm, float eps,
                                  const sk_bf16* W, int64_t ldw, int64_t* ids, float* maxv, int M, int V, int K,
                                  const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream) {
  Handoff h{nullptr, nullptr, 0, const_cast<float*>(sq), w_norm, eps};
  return run_handoff(SK_OP_PRE_LM_ARGMAX, x, ldx, h, W, nullptr, ldw, nullptr, 0, ids, maxv, M, V, K, cfg, ws,
                     ws_bytes, stream);
}

}  // extern "C"
