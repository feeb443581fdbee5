// Internal definitions shared by the HIP backend's host code and kernels.
//
// Device layout of a matrix (written once by BNN_MatrixCreate):
//   tiles = ceil(N / 64); one tile = 64 output features, one per wave lane.
//   wbits [tiles][groups][64] x 16 bytes : the 128 sign bits of (n = 64t + lane, group g),
//                                          byte/bit order as the caller's row (bit k&7 of byte k>>3);
//                                          a wave reading one (t, g) touches 1 KiB contiguously.
//   wscale[tiles][groups][64] fp16 bits  : scale of (n, g); 128 contiguous bytes per (t, g).
//   Features n >= N in the last tile are zero-filled and never stored.
//
// Quantised activation rows (written by the prep kernel into device scratch):
//   planes[row][g][8][4] u32 : bit-plane j, word i, bit b = bit j of Q[g*128 + 32i + b]
//                              (two's complement byte), i.e. 128 bytes per (row, group)
//   sums  [row][g]  i32      : sum of Q over the group
//   rscale[row]     f32      : row scale s (F32 operations)
//   q     [row][K]  i8       : the quantised row itself (matrix-core path)
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "bnn-accelerator.h"
#include "bnn_quant.h"

namespace bnnhip {

constexpr uint32_t kGroup = 128;       // weights per scale group (the only size offered)
constexpr uint32_t kMaxFeatures = 8192;
constexpr uint32_t kMaxGroups = kMaxFeatures / kGroup;
constexpr uint32_t kTile = 64;         // output features per tile
constexpr uint32_t kPlaneWords = 32;   // 8 planes x 4 words per (row, group)
constexpr uint32_t kDotWaves = 4;      // waves per dot workgroup (they split the groups)
// Persistent dot workgroups per CU (tuning constants; overridable at build time).
#ifndef BNN_DOT_WGS_PER_CU_SMALL
#define BNN_DOT_WGS_PER_CU_SMALL 7  // K <= 2048: 71 VGPRs -> 7 waves per SIMD
#endif
#ifndef BNN_DOT_WGS_PER_CU_LARGE
#define BNN_DOT_WGS_PER_CU_LARGE 2  // K > 2048
#endif
constexpr uint32_t kDotWgsPerCuSmall = BNN_DOT_WGS_PER_CU_SMALL;
constexpr uint32_t kDotWgsPerCuLarge = BNN_DOT_WGS_PER_CU_LARGE;

enum KernelKind { KK_PREP = 0, KK_DOT = 1, KK_SCATTER = 2, KK_GEMM = 3, KK_COUNT = 4 };

// Output interpretation of the group-dot kernel.
enum DotMode : int {
    MODE_DOT_I16 = 0,   // store D as int16 [n][g]
    MODE_SUM = 1,       // store Z = sum_g scale*D
    MODE_SUM_SCALED = 2 // store Z * s
};

// One activation block for the prep kernel.  In a batch, block b of the prep
// grid serves row (b - first_block) of the job found through the block table.
struct PrepJob {
    const unsigned char* in;  // logical row 0
    uint64_t in_stride;       // bytes
    uint32_t* planes;         // [rows][groups][32]
    int32_t* sums;            // [rows][groups]
    float* rscale;            // [rows]
    int8_t* q;                // [rows][k] or null
    uint32_t k;
    uint32_t rows;
    int32_t f32;              // F32 input (else I8)
    int32_t aligned;          // F32 rows 4-byte aligned
    uint32_t first_block;
    uint32_t pad_;
};

// One group-dot job.  Work item i of the job is (row, tile) = divmod(i, tiles);
// in a table-mapped batch the job's items start at first_block.
struct DotJob {
    const uint4* wbits;
    const uint16_t* wscale;
    const uint32_t* planes;
    const int32_t* sums;
    const float* rscale;
    unsigned char* out;       // logical row 0 (4-byte aligned for F32, 2 for I16)
    uint64_t out_stride;
    uint32_t n;
    uint32_t groups;
    uint32_t tiles;
    uint32_t rows;
    int32_t mode;
    uint32_t first_block;
};

// One multi-row job on the matrix cores (rows >= kMfmaMinRows), read from the
// matrix's resident layout (sign bits unpacked in LDS by the kernel).
struct GemmJob {
    const uint4* wbits;       // matrix layout [tiles][groups][64] x 16 bytes
    const uint16_t* wscale;   // matrix layout [tiles][groups][64]
    const int8_t* q;          // [rows][k] quantised rows
    const float* rscale;      // [rows]
    unsigned char* out;       // logical row 0 (4-byte aligned for F32, 2 for I16)
    uint64_t out_stride;
    uint32_t n, k, groups, tiles;  // tiles of 64 features, as in the matrix layout
    uint32_t rows;
    int32_t mode;
};

// Rows from which a job runs on the matrix cores instead of the bit-plane kernel.
#ifndef BNN_MFMA_MIN_ROWS
#define BNN_MFMA_MIN_ROWS 8
#endif
constexpr uint32_t kMfmaMinRows = BNN_MFMA_MIN_ROWS;

// Fused batches (bnn_fused.hip): GEMV_F32 jobs sharing one input row produced on
// the device by a pre-operation.  One entry per job; the job's tiles are the
// workgroups first_tile .. first_tile + tiles - 1 of the launch.
// PRE_ROW_I8: the row is int8 (GEMV / DOT_GROUPS input: checked for -128, used as Q
// with row scale 1; single jobs only)
enum PreKind : int32_t { PRE_ROW = 0, PRE_RMSNORM = 1, PRE_SILU_MUL = 2, PRE_ROW_I8 = 3 };
constexpr uint32_t kFusedMaxWidth = 6144;  // K of a fused batch (LDS holds the whole row)
constexpr uint32_t kFusedInline = 3;       // jobs passed in the kernel arguments

struct FusedJob {
    const uint4* wbits;
    const uint16_t* wscale;
    float* out;  // output row
    uint32_t n, tiles, first_tile;
    uint32_t post_off;  // POST_SILU_MUL, first job of a pair: offset of its rows in post_out
};

// Operation on pairs of outputs of a fused batch: with POST_SILU_MUL the 2m jobs are
// m pairs (job p, job m + p) of equal n, and post_out receives y_p / (1 + expf(-y_p)) * y_(m+p).
enum PostKind : int32_t { POST_NONE = 0, POST_SILU_MUL = 1 };

struct FusedArgs {
    const FusedJob* jobs;  // device table, or null: the one job is `single`
    uint32_t njobs;
    int32_t kind;          // PreKind
    uint32_t width;        // K
    float eps;
    const float* a;        // RMSNORM: x; SILU_MUL: gate
    const float* b;        // RMSNORM: residual (may be null); SILU_MUL: up
    const float* gain;     // RMSNORM
    float* a_out;          // RMSNORM: receives x + residual (may be null)
    const float* row;      // ROW: the input row
    int32_t* err;          // set to err_code when the RMSNORM check fails (may be null)
    int32_t err_code;
    int32_t post;          // PostKind
    float* post_out;       // POST_SILU_MUL
    // the jobs themselves, in the kernel arguments, when there are at most kFusedInline
    // (inline_jobs != 0; a single job: jobs == null): the first tile's weight loads then
    // wait for no table read
    FusedJob inl[kFusedInline];
    uint32_t inline_jobs;
    // when every walked job (or pair) j starts at tile j << walk_shift, the job of tile t is
    // min(t >> walk_shift, last); 32: none does, the kernel walks the table
    uint32_t walk_shift;
    float* mirror;         // single F32 job: host memory that also receives the output row (may be null)
    int32_t dot_out;       // DOT_GROUPS: out receives int16 D[n][group] instead of the sums
    // single job: completion signal (may be null).  Workgroup b stores seq into the pinned
    // host word done_flags[b] once its results are visible system-wide.
    uint64_t* done_flags;
};

// Pinned host words of a device (bnn_accel_device::status_host): [0] seq of the last
// synchronous call that met an illegal input, [1] the same for asynchronous launches,
// then from kDoneFlagWord one completion word per workgroup of a single-row launch.
constexpr uint32_t kDoneFlagWord = 32;     // 256 bytes in
constexpr uint32_t kDoneFlagSlots = 1024;  // workgroups a single-row launch may signal with
constexpr size_t kStatusHostBytes = (kDoneFlagWord + kDoneFlagSlots) * sizeof(uint64_t);

// Kernel timing: when `start` is set, the next kernel launched through launch_kernel
// records its own start and end into these events (taken from the dispatch itself,
// so timing adds no packet between kernels); the launch clears them.
struct LaunchEvents {
    hipEvent_t start, stop;
};
extern thread_local LaunchEvents t_launch_events;

template <typename F, typename... Args>
inline void launch_kernel(F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t stream, Args... args) {
    if (t_launch_events.start != nullptr) {
        const LaunchEvents ev = t_launch_events;
        t_launch_events = LaunchEvents{nullptr, nullptr};
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, ev.start, ev.stop, 0u, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream, args...);
    }
}

// Host-side launchers (bnn_kernels.hip).  All are asynchronous on `stream`.
// Single job: descriptor passed by value.  `validate_only` runs only the
// legality pass of prep (over all rows of a job processed in several chunks).
hipError_t launch_prep(hipStream_t stream, const PrepJob& job, bool validate_only, uint64_t seq,
                       uint64_t* flag, uint64_t* host_status);
hipError_t launch_dot(hipStream_t stream, const DotJob& job, uint32_t cu_count, uint64_t seq,
                      const uint64_t* flag);
// Work items of the dot kernel for a job (rows x groups of tiles); in a batch the
// tiles per item follow the batch's largest group count.
uint32_t dot_items(uint32_t tiles, uint32_t rows, uint32_t max_groups);
// Batch: device-resident job tables.  Prep: one block per row, block -> job map.
// Dot: items = sum of rows*tiles; job of an item = item / uniform_items when every
// job has that many items, else item_job[item].
hipError_t launch_prep_batch(hipStream_t stream, const PrepJob* jobs, const uint32_t* block_job,
                             uint32_t blocks, uint32_t max_groups, uint64_t seq, uint64_t* flag,
                             uint64_t* host_status);
// `scales`: some job sums scaled products; false for batches of DOT_GROUPS jobs only,
// which then read no scales.
hipError_t launch_dot_batch(hipStream_t stream, const DotJob* jobs, const uint32_t* item_job, uint32_t items,
                            uint32_t uniform_items, uint32_t max_groups, bool scales, uint32_t cu_count,
                            uint64_t seq, const uint64_t* flag);
hipError_t launch_gemm(hipStream_t stream, const GemmJob& job, uint32_t cu_count, uint64_t seq,
                       const uint64_t* flag);
// One launch of a fused batch of `tiles` 64-feature tiles on `grid` workgroups
// (bnn_fused.hip).
hipError_t launch_fused(hipStream_t stream, const FusedArgs& args, uint32_t tiles, uint32_t grid, uint64_t seq,
                        uint64_t* flag, uint64_t* host_status);
// One layer of a chained batch (BNNX_BatchCreateChain): a GEMM_F32 matrix and the
// optional mapping of its outputs, out = post_scale * y + post_bias, then ReLU.
struct ChainLayer {
    const uint4* wbits;       // matrix layout [tiles][groups][64] x 16 bytes
    const uint16_t* wscale;   // [tiles][groups][64]
    const float* post_scale;  // [n], or null: no affine mapping
    const float* post_bias;   // [n] (set with post_scale)
    uint32_t k, n, groups, tiles;
    int32_t relu;
    uint32_t pad_;
};
constexpr uint32_t kChainMaxLayers = 16;
constexpr uint32_t kChainMaxWidth = 4096;  // widest layer input or output
constexpr uint32_t kChainMaxRows = 4096;
static_assert(sizeof(ChainLayer) % 4 == 0 && kChainMaxLayers * sizeof(ChainLayer) / 4 <= 1024,
              "the chain kernel copies the layer table with one word per thread");
struct ChainArgs {
    const ChainLayer* layers;  // device table of `count` layers
    uint32_t count, rows;
    uint32_t k0;               // layer 0's input width
    uint32_t pad_;
    const unsigned char* in;   // row 0 of the input view (F32, 4-byte aligned)
    uint64_t in_stride;
    unsigned char* out;        // row 0 of the output view (F32, 4-byte aligned)
    uint64_t out_stride;
};
// One launch of a chained batch: a workgroup per row (bnn_chain.hip).
hipError_t launch_chain(hipStream_t stream, const ChainArgs& args, uint64_t seq, uint64_t* flag,
                        uint64_t* host_status);
hipError_t launch_scatter(hipStream_t stream, const unsigned char* src, size_t src_stride,
                          unsigned char* dst, size_t dst_stride, size_t row_bytes, uint32_t rows,
                          uint64_t seq, const uint64_t* flag);

}  // namespace bnnhip

struct bnn_accel_device {
    int ordinal;
    uint32_t cu_count;
    hipStream_t stream;
    size_t live_matrices;
    size_t live_buffers;
    size_t live_batches;       // prepared batches (extension API)
    uint64_t seq;              // job sequence number, never 0 for a launched job
    uint64_t async_first_seq;  // first seq launched asynchronously since the last synchronise (0: none)
    uint64_t retired;          // matrices and buffers destroyed so far
    uint64_t* flag_dev;        // device word [0]: seq of the last job that met an illegal input
    // pinned host words written by the kernels (kStatusHostBytes): [0] seq of the last
    // synchronous call that met an illegal input, [1] the same for asynchronous launches
    // (read by BNNX_DeviceSynchronize), from kDoneFlagWord the completion words of the
    // workgroups of single-row launches
    uint64_t* status_host;
    unsigned char* scratch;    // grow-only device scratch
    size_t scratch_bytes;
    unsigned char* static_scratch;  // this GPU's fixed scratch array (BNNX_ExecuteNoAlloc)
    unsigned char* pinned;     // grow-only pinned host staging for transfers
    size_t pinned_bytes;
    unsigned char* wring;      // pinned ring for small writes, copied asynchronously on `stream`
    size_t wring_off;          // next free byte; the ring restarts after a stream synchronisation
    // Host mirror of the last single-row BNN_Execute output: the fused kernel also writes
    // the row into this pinned memory, so a BNN_BufferRead of (part of) that output right
    // after the call is a host copy.  Any other call that could change buffers drops it.
    float* mirror;             // pinned, kMaxFeatures floats
    BNN_Buffer mirror_buf;     // null: no valid mirror
    size_t mirror_off, mirror_bytes;
    unsigned char* table_host; // grow-only pinned staging for batch job tables
    size_t table_host_bytes;
    unsigned char* table_dev;  // grow-only device copy of the batch job tables
    size_t table_dev_bytes;
    // Resource generation: bumped by every matrix/buffer create or destroy and by
    // every scratch reallocation, i.e. whenever a device pointer could change.
    uint64_t generation;
    // The last batch whose tables sit in table_dev (reused for an identical batch
    // of the same generation).
    BNN_Job* batch_jobs;
    uint32_t batch_count, batch_cap;
    uint64_t batch_generation;
    uint32_t batch_prep_blocks, batch_items, batch_uniform_items, batch_max_groups;
    size_t batch_prep_tab, batch_dot_tab, batch_prep_map, batch_tables;
    bool batch_needs_nearest;  // some job of the cached batch is an FP32 operation
    // optional kernel timing (extension API): event pairs recorded around
    // launches, resolved after the call's synchronisation
    int timing;
    bool events_created;       // the event pairs exist (made by the first BNNX_KernelTiming(.., 1))
    static constexpr int kTimingSlots = 1024;
    hipEvent_t ev_begin[kTimingSlots], ev_end[kTimingSlots];
    int ev_kind[kTimingSlots];
    int ev_used;
    double kernel_ms[bnnhip::KK_COUNT];
    uint64_t kernel_launches[bnnhip::KK_COUNT];
};

struct bnn_accel_matrix {
    BNN_Device device;
    uint32_t k, n, groups, tiles;
    uint4* wbits;
    uint16_t* wscale;
};

// A prepared batch: job tables and the rows' scratch in one device allocation,
// built once; every launch is two kernel launches and nothing else.
struct bnnx_batch {
    BNN_Device device;
    uint64_t retired;  // device->retired when built: valid while no matrix or buffer was destroyed since
    unsigned char* mem;
    uint32_t prep_blocks, items, uniform_items, max_groups;
    size_t prep_tab, dot_tab, prep_map;
    bool needs_nearest;
    // fused batch (BNNX_BatchCreateFused): one launch of `fused_tiles` workgroups
    bool fused;
    uint32_t fused_tiles, fused_grid;
    bnnhip::FusedArgs fused_args;  // jobs points into mem
    // chained batch (BNNX_BatchCreateChain): one launch of a workgroup per row
    bool chain;
    bnnhip::ChainArgs chain_args;  // layers points into mem
};

struct bnn_accel_buffer {
    BNN_Device device;
    size_t size;
    unsigned char* dev;
    bool exposed;  // its device pointer was handed out (BNNX_BufferDevicePointer): never mirrored
};
