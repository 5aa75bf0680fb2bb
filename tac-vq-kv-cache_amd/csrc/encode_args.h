// Argument block shared by the encode kernels (encode.hip, encode_full.hip).
#pragma once

#include "jkv_common.h"

namespace jkv {

struct EncodeArgs {
  const void* states;
  int64_t sb, sh, st;  // element strides of the B, H, T axes
  int64_t B, H, T, G, d, S, K;
  const float* tables;      // fp32 masters [P,S,K,d]
  const float* sel_tables;  // whitened selector tables [P,S,K,d] or null
  const float* whiteners;   // [P,d,d] or null
  uint8_t* codes;
  int64_t cb, ch, ct;  // byte strides of the B, H, T axes
  int32_t n_exits;
  int32_t exit_depth[JKV_MAX_EXITS];
  void* recon[JKV_MAX_EXITS];
};

// Full-vector residual VQ (d = 128, K = 256) on MFMA: workspace it needs for
// P problems of S stages (without and with an assignment whitener) and its
// launch (whitened when a.whiteners is set).
int64_t full_workspace_bytes(int64_t P, int64_t S);
int64_t full_wh_workspace_bytes(int64_t P, int64_t S);  // with an assignment whitener
int launch_full(const EncodeArgs& a, void* workspace, hipStream_t stream);
// The same for n <= 64 jobs of one geometry (no whitener, at most two
// exits) in one table launch and one search launch; `workspace` holds n
// regions of full_workspace_bytes(P, S).
int launch_full_many(const EncodeArgs* jobs, int n, void* workspace, hipStream_t stream);

// Grouped encode on MFMA (d in {4, 8}, K = 256, S <= 2, fp16 states): one job
// is one encode call; a launch runs one or two jobs of the same geometry (a
// token's K and V).  Logical workgroups below `split` take job 0.
struct MfmaJob {
  EncodeArgs e;
  void* recon_depth[2];  // reconstruction at depth 1 / 2 (or null)
  int64_t rows_per_wg;
  int64_t n_chunks;      // row chunks per problem
};
struct MfmaArgs {
  MfmaJob job[2];
  int64_t split;
};

// Many jobs of one geometry in one launch (every layer's K and V of a
// cache): the geometry once, then each job's buffers.  Job j takes logical
// workgroups [j * per_job, (j + 1) * per_job).
static const int kMaxManyJobs = 64;
struct MfmaJobBuffers {
  const void* states;
  const float* tables;
  uint8_t* codes;
  void* recon_depth[2];
};
struct MfmaManyArgs {
  MfmaJob shape;  // geometry, strides and row chunks (its buffers unused)
  int64_t per_job;
  int32_t n_jobs;
  MfmaJobBuffers buf[kMaxManyJobs];
};

// Rows a workgroup encodes per iteration (4 waves x 64 rows).
static const int kGroupedRowsPerIter = 256;

// Unwhitened grouped encode (encode_grouped.hip); e2 = second job or null.
int launch_grouped(const EncodeArgs& e, const EncodeArgs* e2, hipStream_t stream);
// The same for n <= kMaxManyJobs jobs that share everything but their
// buffers (states, tables, codes, reconstructions).
int launch_grouped_many(const EncodeArgs* jobs, int n, hipStream_t stream);

}  // namespace jkv
