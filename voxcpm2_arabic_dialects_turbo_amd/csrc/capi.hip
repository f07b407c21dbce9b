// C-ABI entry points of libvoxattn.so (declared in include/vox_attn.h).
//
// Every entry point validates its arguments on the host, launches on the caller's stream, checks the launch, and
// returns a status (VOX_OK, VOX_EINVAL, VOX_EHIP) instead of throwing; vox_last_error() gives the calling thread's
// message for the last failure. Nothing here allocates, frees or synchronizes, so every call can be captured into
// a HIP graph.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "vox_kernels.h"
#include "../../include/vox_attn.h"

namespace {

thread_local char g_err[512] = "";
int g_decode_grid_override = 0;

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return VOX_OK;
  return fail(VOX_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }


constexpr int kHeadDim = 128;
constexpr int kMaxHeads = 16;

}  // namespace

extern "C" {

const char* vox_last_error(void) { return g_err; }

int vox_abi_version(void) { return VOX_ABI_VERSION; }

int vox_store_kvcache(const void* key, const void* value, int64_t key_row_stride, int64_t value_row_stride,
                      void* k_cache, void* v_cache, int64_t num_slots, const int32_t* slot_mapping,
                      int64_t num_tokens, int num_kv_heads, int head_dim, void* stream) {
  if (num_tokens < 0) return fail(VOX_EINVAL, "store_kvcache: num_tokens %lld < 0", (long long)num_tokens);
  if (num_tokens == 0) return VOX_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return fail(VOX_EINVAL, "store_kvcache: null pointer argument");
  if (num_kv_heads <= 0 || head_dim <= 0) return fail(VOX_EINVAL, "store_kvcache: bad head shape");
  if (num_slots <= 0) return fail(VOX_EINVAL, "store_kvcache: empty cache");
  const int row = num_kv_heads * head_dim;
  if (key_row_stride < row || value_row_stride < row)
    return fail(VOX_EINVAL, "store_kvcache: row stride smaller than num_kv_heads * head_dim");
  const bool vec16 = (row % 8 == 0) && (key_row_stride % 8 == 0) && (value_row_stride % 8 == 0) &&
                     aligned16(key) && aligned16(value) && aligned16(k_cache) && aligned16(v_cache);
  return hip_status(vox::launch_store_kvcache(key, value, key_row_stride, value_row_stride, k_cache, v_cache,
                                              num_slots, slot_mapping, num_tokens, row, vec16,
                                              (hipStream_t)stream),
                    "store_kvcache launch");
}

int vox_decode_workgroups(void) {
  if (g_decode_grid_override > 0) return g_decode_grid_override;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    cus = 256;  // MI355X
  }
  return cus;  // one 4-wave workgroup per CU: the split kernel's ranges are balanced over every CU
}

void vox_set_decode_workgroups(int workgroups) { g_decode_grid_override = workgroups > 0 ? workgroups : 0; }

namespace {
// Workspace of decode launches of up to `slice` sequences over `grid` workgroups, each part 256-byte aligned: the fp32
// split-KV partials [slice + grid][kPartialFloats], the int32 step layout [slice + 2] (first step of every sequence,
// the total, the active workgroup count) that the merge kernel reads, then the plan records [grid][kPlanRecInts].
struct DecodeWorkspace {
  size_t partials, steps, plan, total;
};
size_t round256(size_t n) { return (n + 255) / 256 * 256; }
DecodeWorkspace decode_workspace(int slice, int grid) {
  DecodeWorkspace w;
  w.partials = 0;
  w.steps = round256((size_t)(slice + grid) * vox::kPartialFloats * 4);
  w.plan = w.steps + round256((size_t)(slice + 2) * 4);
  w.total = w.plan + round256((size_t)grid * vox::kPlanRecInts * 4);
  return w;
}
}  // namespace

size_t vox_decode_workspace_bytes(int batch) {
  if (batch <= 0) return 0;
  const int slice = batch < vox::kMaxSeqPerLaunch ? batch : vox::kMaxSeqPerLaunch;
  return decode_workspace(slice, vox_decode_workgroups()).total;
}

}  // extern "C"

namespace {
// Launches the decode kernel over `batch` sequences in slices of kMaxSeqPerLaunch (each slice's step layout lives
// in LDS), all sharing the workspace; `a` describes the whole batch. A call of several slices runs unplanned (the
// workspace holds one plan).
// a's split-KV scratch and plan records in the workspace, for launches of up to `slice` sequences
vox::DecodeArgs with_workspace(const vox::DecodeArgs& a, int slice, int plan_mode, void* workspace) {
  const DecodeWorkspace ws = decode_workspace(slice, a.grid);
  vox::DecodeArgs d = a;
  d.partials = (float*)((char*)workspace + ws.partials);
  d.steps = (int32_t*)((char*)workspace + ws.steps);
  d.plan = (int32_t*)((char*)workspace + ws.plan);
  d.plan_mode = plan_mode;
  return d;
}

int launch_decode_slices(const vox::DecodeArgs& a, int batch, int num_kv_heads, int plan, void* workspace,
                         hipStream_t stream) {
  const int slice_max = batch < vox::kMaxSeqPerLaunch ? batch : vox::kMaxSeqPerLaunch;
  const vox::DecodeArgs base =
      with_workspace(a, slice_max, batch <= vox::kMaxSeqPerLaunch ? plan : vox::kPlanNone, workspace);
  for (int b0 = 0; b0 < batch; b0 += vox::kMaxSeqPerLaunch) {
    vox::DecodeArgs s = base;
    s.batch = batch - b0 < vox::kMaxSeqPerLaunch ? batch - b0 : vox::kMaxSeqPerLaunch;
    s.block_tables = base.block_tables + (int64_t)b0 * base.bt_stride;
    if (base.cu_q) {  // varlen: rows are absolute (cu_seqlens_q), only the sequence arrays move
      s.cu_q = base.cu_q + b0;
      s.cu_k = base.cu_k + b0;
    } else {
      s.q = base.q + (int64_t)b0 * base.q_row_stride;
      s.context_lens = base.context_lens + b0;
      s.out = base.out + (int64_t)b0 * base.out_row_stride;
      if (base.slot_mapping) {
        s.slot_mapping = base.slot_mapping + b0;
        s.new_k = base.new_k + (int64_t)b0 * base.new_k_stride;
        s.new_v = base.new_v + (int64_t)b0 * base.new_v_stride;
      }
    }
    const int st = hip_status(vox::launch_decode(s, num_kv_heads, stream), "decode launch");
    if (st != VOX_OK) return st;
  }
  return VOX_OK;
}
}  // namespace

extern "C" {

}  // extern "C"

namespace {
// Validates a decode call's arguments (batch > 0) and fills its launch descriptor.
int decode_setup(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache, int64_t num_blocks,
                 int block_size, const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                 const int32_t* context_lens, int batch, int num_heads, int num_kv_heads, int head_dim,
                 float softmax_scale, void* workspace, size_t workspace_bytes, void* out, vox::DecodeArgs* out_args) {
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out)
    return fail(VOX_EINVAL, "decode_attn: null pointer argument");
  if (head_dim != kHeadDim) return fail(VOX_EINVAL, "decode_attn: head_dim %d unsupported (128 only)", head_dim);
  if (num_kv_heads != 1 && num_kv_heads != 2)
    return fail(VOX_EINVAL, "decode_attn: num_kv_heads %d unsupported (1 or 2)", num_kv_heads);
  if (num_heads <= 0 || num_heads > kMaxHeads || num_heads % num_kv_heads)
    return fail(VOX_EINVAL, "decode_attn: num_heads %d must be <= 16 and a multiple of num_kv_heads", num_heads);
  if (block_size <= 0 || block_size % 32)
    return fail(VOX_EINVAL, "decode_attn: block_size %d must be a positive multiple of 32", block_size);
  if (max_blocks <= 0 || bt_stride < max_blocks) return fail(VOX_EINVAL, "decode_attn: bad block table shape");
  if (num_blocks <= 0) return fail(VOX_EINVAL, "decode_attn: empty cache");
  if (q_row_stride < (int64_t)num_heads * head_dim || q_row_stride % 8)
    return fail(VOX_EINVAL, "decode_attn: q row stride %lld", (long long)q_row_stride);
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out) || !aligned16(workspace))
    return fail(VOX_EINVAL, "decode_attn: q, caches, out and workspace must be 16-byte aligned");
  if (!std::isfinite(softmax_scale)) return fail(VOX_EINVAL, "decode_attn: softmax_scale is not finite");
  if ((int64_t)max_blocks * block_size > (1 << 30)) return fail(VOX_EINVAL, "decode_attn: block table too wide");
  const int grid = vox_decode_workgroups();
  const size_t need = vox_decode_workspace_bytes(batch);
  if (workspace_bytes < need || !workspace)
    return fail(VOX_EINVAL, "decode_attn: workspace of %zu bytes, %zu needed", workspace_bytes, need);

  vox::DecodeArgs& a = *out_args;
  a = vox::DecodeArgs{};
  a.q = (const uint16_t*)q;
  a.q_row_stride = q_row_stride;
  a.k_cache = (const uint16_t*)k_cache;
  a.v_cache = (const uint16_t*)v_cache;
  a.num_blocks = num_blocks;
  a.block_size = block_size;
  a.block_tables = block_tables;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks;
  a.context_lens = context_lens;
  a.batch = batch;
  a.num_heads = num_heads;
  a.group = num_heads / num_kv_heads;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.grid = grid;
  a.out = (uint16_t*)out;
  a.out_row_stride = (int64_t)num_heads * head_dim;
  return VOX_OK;
}
}  // namespace

extern "C" {

int vox_decode_attn(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                    int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                    int max_blocks, const int32_t* context_lens, int batch, int num_heads, int num_kv_heads,
                    int head_dim, float softmax_scale, int plan, void* workspace, size_t workspace_bytes,
                    void* out, void* stream) {
  if (batch < 0) return fail(VOX_EINVAL, "decode_attn: batch < 0");
  if (plan != VOX_PLAN_NONE && plan != VOX_PLAN_RECORD && plan != VOX_PLAN_REUSE)
    return fail(VOX_EINVAL, "decode_attn: plan mode %d", plan);
  if (batch == 0) return VOX_OK;
  vox::DecodeArgs a;
  const int st = decode_setup(q, q_row_stride, k_cache, v_cache, num_blocks, block_size, block_tables, bt_stride,
                              max_blocks, context_lens, batch, num_heads, num_kv_heads, head_dim, softmax_scale,
                              workspace, workspace_bytes, out, &a);
  if (st != VOX_OK) return st;
  // batches beyond one launch's LDS step layout run as consecutive launches on the stream (shared workspace)
  return launch_decode_slices(a, batch, num_kv_heads, plan, workspace, (hipStream_t)stream);
}

int vox_decode_attn_store(const void* q, int64_t q_row_stride, const void* key, const void* value,
                          int64_t key_row_stride, int64_t value_row_stride, const int32_t* slot_mapping,
                          void* k_cache, void* v_cache, int64_t num_blocks, int block_size,
                          const int32_t* block_tables, int64_t bt_stride, int max_blocks, const int32_t* context_lens,
                          int batch, int num_heads, int num_kv_heads, int head_dim, float softmax_scale, int plan,
                          void* workspace, size_t workspace_bytes, void* out, void* stream) {
  if (batch < 0) return fail(VOX_EINVAL, "decode_attn_store: batch < 0");
  if (plan != VOX_PLAN_NONE && plan != VOX_PLAN_RECORD && plan != VOX_PLAN_REUSE)
    return fail(VOX_EINVAL, "decode_attn_store: plan mode %d", plan);
  if (batch == 0) return VOX_OK;
  if (!key || !value || !slot_mapping) return fail(VOX_EINVAL, "decode_attn_store: null key, value or slot_mapping");
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (key_row_stride < row || value_row_stride < row || key_row_stride % 8 || value_row_stride % 8 ||
      !aligned16(key) || !aligned16(value))
    return fail(VOX_EINVAL, "decode_attn_store: key / value rows must be 16-byte aligned, strides multiples of 8 "
                            "elements and at least num_kv_heads * head_dim");
  vox::DecodeArgs a;
  const int st = decode_setup(q, q_row_stride, k_cache, v_cache, num_blocks, block_size, block_tables, bt_stride,
                              max_blocks, context_lens, batch, num_heads, num_kv_heads, head_dim, softmax_scale,
                              workspace, workspace_bytes, out, &a);
  if (st != VOX_OK) return st;
  a.slot_mapping = slot_mapping;
  a.new_k = (const uint16_t*)key;
  a.new_v = (const uint16_t*)value;
  a.new_k_stride = key_row_stride;
  a.new_v_stride = value_row_stride;
  return launch_decode_slices(a, batch, num_kv_heads, plan, workspace, (hipStream_t)stream);
}

size_t vox_prefill_workspace_bytes(int batch) { return vox_decode_workspace_bytes(batch); }

}  // extern "C"

// ---- allocation-free decode: the split-KV scratch in a static device array ----------------------------------------
//
// vox_decode_attn_noalloc serves callers that cannot allocate (code under HIP graph capture that must not touch an
// allocator, tight serving loops): the workspace vox_decode_attn takes as an argument lives in `scratch`, a
// file-scope device array that every GPU the library runs on holds until the process ends. In host code `scratch`
// names a host-side stand-in, not the device array: its device address on each GPU comes from hipGetSymbolAddress,
// looked up once per device with that device current, and only that address is handed to kernels.
namespace {
constexpr int kMaxDevices = 64;
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// This device's address of `scratch` (nullptr and an error message on failure).
void* scratch_on_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    fail(VOX_EHIP, "decode_attn_noalloc: no current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      fail(VOX_EHIP, "decode_attn_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" {

int vox_decode_attn_noalloc(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                            int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                            int max_blocks, const int32_t* context_lens, int batch, int num_heads, int num_kv_heads,
                            int head_dim, float softmax_scale, void* out, void* stream) {
  if (batch < 0) return fail(VOX_EINVAL, "decode_attn_noalloc: batch < 0");
  if (batch == 0) return VOX_OK;
  const size_t need = vox_decode_workspace_bytes(batch);
  if (need > kScratchBytes)
    return fail(VOX_EINVAL, "decode_attn_noalloc: needs %zu bytes of scratch, the static array holds %zu", need,
                kScratchBytes);
  void* ws = scratch_on_current_device();
  if (!ws) return VOX_EHIP;
  return vox_decode_attn(q, q_row_stride, k_cache, v_cache, num_blocks, block_size, block_tables, bt_stride,
                         max_blocks, context_lens, batch, num_heads, num_kv_heads, head_dim, softmax_scale,
                         VOX_PLAN_NONE, ws, kScratchBytes, out, stream);
}

}  // extern "C"

namespace {
// Validates a prefill call's shared arguments (all but the output) and fills its launch descriptor.
int prefill_setup(const char* fn, const void* q, int64_t q_row_stride, const void* key, const void* value,
                  int64_t key_row_stride, int64_t value_row_stride, const void* k_cache, const void* v_cache,
                  int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch, int max_seqlen_q,
                  int uniform_seqlen_q, int uniform_seqlen_k, int num_heads, int num_kv_heads, int head_dim,
                  float softmax_scale, int causal, vox::PrefillArgs* a) {
  if (!q) return fail(VOX_EINVAL, "%s: null q", fn);
  if (head_dim != kHeadDim) return fail(VOX_EINVAL, "%s: head_dim %d unsupported (128 only)", fn, head_dim);
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads)
    return fail(VOX_EINVAL, "%s: num_heads %d not a multiple of num_kv_heads %d", fn, num_heads, num_kv_heads);
  const int group = num_heads / num_kv_heads;
  if (128 % group) return fail(VOX_EINVAL, "%s: group size %d must divide 128", fn, group);
  if ((cu_seqlens_q == nullptr) != (cu_seqlens_k == nullptr))
    return fail(VOX_EINVAL, "%s: give both cu_seqlens or neither", fn);
  if (!cu_seqlens_q && (uniform_seqlen_q <= 0 || uniform_seqlen_k <= 0))
    return fail(VOX_EINVAL, "%s: uniform lengths must be positive without cu_seqlens", fn);
  if (!cu_seqlens_q && max_seqlen_q != uniform_seqlen_q)
    return fail(VOX_EINVAL, "%s: max_seqlen_q must equal the uniform length", fn);
  if (q_row_stride < (int64_t)num_heads * head_dim || q_row_stride % 8 || !aligned16(q))
    return fail(VOX_EINVAL, "%s: q must be 16-byte aligned with a row stride >= H*D, multiple of 8", fn);
  if (!std::isfinite(softmax_scale)) return fail(VOX_EINVAL, "%s: softmax_scale is not finite", fn);
  if (block_tables) {
    if (!k_cache || !v_cache) return fail(VOX_EINVAL, "%s: block tables without caches", fn);
    if (block_size <= 0 || max_blocks <= 0 || bt_stride < max_blocks || num_blocks <= 0)
      return fail(VOX_EINVAL, "%s: bad block table or cache shape", fn);
    if (!aligned16(k_cache) || !aligned16(v_cache)) return fail(VOX_EINVAL, "%s: caches not aligned", fn);
  } else {
    if (!key || !value) return fail(VOX_EINVAL, "%s: null key/value without block tables", fn);
    if (key_row_stride < (int64_t)num_kv_heads * head_dim || value_row_stride < (int64_t)num_kv_heads * head_dim ||
        key_row_stride % 8 || value_row_stride % 8 || !aligned16(key) || !aligned16(value))
      return fail(VOX_EINVAL, "%s: key/value must be 16-byte aligned rows, stride multiple of 8", fn);
    if (key_row_stride >= (1 << 24) || value_row_stride >= (1 << 24))
      return fail(VOX_EINVAL, "%s: key/value row stride must be below 2^24 elements", fn);
  }
  *a = vox::PrefillArgs{};
  a->q = (const uint16_t*)q;
  a->q_row_stride = q_row_stride;
  a->k_src = (const uint16_t*)key;
  a->v_src = (const uint16_t*)value;
  a->k_row_stride = key_row_stride;
  a->v_row_stride = value_row_stride;
  a->k_cache = (const uint16_t*)k_cache;
  a->v_cache = (const uint16_t*)v_cache;
  a->num_blocks = num_blocks;
  a->block_size = block_size;
  a->block_tables = block_tables;
  a->bt_stride = bt_stride;
  a->max_blocks = max_blocks;
  a->cu_q = cu_seqlens_q;
  a->cu_k = cu_seqlens_k;
  a->uniform_q = uniform_seqlen_q;
  a->uniform_k = uniform_seqlen_k;
  a->batch = batch;
  a->num_heads = num_heads;
  a->num_kv_heads = num_kv_heads;
  a->group = group;
  a->scale_log2 = softmax_scale * 1.4426950408889634f;
  a->causal = causal ? 1 : 0;
  return VOX_OK;
}

// Whether a varlen call's one-query rows can run on the split-KV decode kernels (paged keys, cu_seqlens, the
// decode kernels' head and block shapes, an output the merge kernel can write with 16-byte stores, the workspace).
bool varlen_decode_rows(const vox::PrefillArgs& a, const void* workspace, int num_kv_heads) {
  return workspace && a.block_tables && a.cu_q && a.num_heads <= kMaxHeads && (num_kv_heads == 1 || num_kv_heads == 2) &&
         a.block_size % 32 == 0 && (int64_t)a.max_blocks * a.block_size <= (1 << 30) && a.out_row_stride % 8 == 0 &&
         ((uintptr_t)a.out & 15u) == 0;
}
int check_varlen_workspace(const char* fn, int batch, int plan, const void* workspace, size_t workspace_bytes) {
  const size_t need = vox_prefill_workspace_bytes(batch);
  if (workspace_bytes < need || !aligned16(workspace))
    return fail(VOX_EINVAL, "%s: workspace of %zu bytes (16-byte aligned), %zu needed", fn, workspace_bytes, need);
  if (plan != VOX_PLAN_NONE && plan != VOX_PLAN_RECORD && plan != VOX_PLAN_REUSE)
    return fail(VOX_EINVAL, "%s: plan mode %d", fn, plan);
  return VOX_OK;
}
// the decode kernels' arguments for the one-query rows of the paged varlen call a (varlen mode: rows from cu_seqlens)
vox::DecodeArgs varlen_decode_args(const vox::PrefillArgs& a, int64_t q_row_stride, int64_t num_blocks, int num_heads,
                                   int num_kv_heads) {
  vox::DecodeArgs d{};
  d.q = a.q;
  d.q_row_stride = q_row_stride;
  d.k_cache = a.k_cache;
  d.v_cache = a.v_cache;
  d.num_blocks = num_blocks;
  d.block_size = a.block_size;
  d.block_tables = a.block_tables;
  d.bt_stride = a.bt_stride;
  d.max_blocks = a.max_blocks;
  d.batch = a.batch;
  d.num_heads = num_heads;
  d.group = num_heads / num_kv_heads;
  d.scale_log2 = a.scale_log2;
  d.grid = vox_decode_workgroups();
  d.out = a.out;
  d.out_row_stride = a.out_row_stride;
  d.cu_q = a.cu_q;
  d.cu_k = a.cu_k;
  return d;
}
}  // namespace

extern "C" {

int vox_prefill_attn(const void* q, int64_t q_row_stride, const void* key, const void* value,
                     int64_t key_row_stride, int64_t value_row_stride, const void* k_cache, const void* v_cache,
                     int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                     int max_blocks, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch,
                     int max_seqlen_q, int uniform_seqlen_q, int uniform_seqlen_k, int num_heads, int num_kv_heads,
                     int head_dim, float softmax_scale, int causal, void* out, int64_t out_row_stride, int plan,
                     void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 0 || max_seqlen_q < 0) return fail(VOX_EINVAL, "prefill_attn: negative batch or max_seqlen_q");
  if (batch == 0 || max_seqlen_q == 0) return VOX_OK;
  if (!out) return fail(VOX_EINVAL, "prefill_attn: null out");
  if (out_row_stride < (int64_t)num_heads * head_dim || out_row_stride % 4 || ((uintptr_t)out & 7u))
    return fail(VOX_EINVAL, "prefill_attn: bad out row stride or alignment");
  vox::PrefillArgs a;
  const int st = prefill_setup("prefill_attn", q, q_row_stride, key, value, key_row_stride, value_row_stride, k_cache,
                               v_cache, num_blocks, block_size, block_tables, bt_stride, max_blocks, cu_seqlens_q,
                               cu_seqlens_k, batch, max_seqlen_q, uniform_seqlen_q, uniform_seqlen_k, num_heads,
                               num_kv_heads, head_dim, softmax_scale, causal, &a);
  if (st != VOX_OK) return st;
  a.out = (uint16_t*)out;
  a.out_row_stride = out_row_stride;
  const hipStream_t s = (hipStream_t)stream;
  // One-query sequences of a paged varlen call (the decode rows of a mixed step) go to the split-KV decode kernels,
  // which spread long contexts over every CU; the prefill kernel takes the rest. Needs the workspace and the decode
  // kernels' shapes; otherwise the prefill kernel takes every row.
  if (varlen_decode_rows(a, workspace, num_kv_heads)) {
    const int sw = check_varlen_workspace("prefill_attn", batch, plan, workspace, workspace_bytes);
    if (sw != VOX_OK) return sw;
    a.skip_single = 1;
    a.persistent = 1;  // the (q tile, sequence) grid would be mostly the decode rows' empty tiles
    const vox::DecodeArgs d = varlen_decode_args(a, q_row_stride, num_blocks, num_heads, num_kv_heads);
    if (max_seqlen_q > 1 && vox::mixed_launch_fits(a, num_kv_heads)) {
      // both kinds of rows in one launch, sharing the CUs (then the merge kernel)
      const vox::DecodeArgs dw = with_workspace(d, batch, plan, workspace);
      return hip_status(vox::launch_mixed(a, max_seqlen_q, dw, num_kv_heads, s), "prefill_attn mixed launch");
    }
    if (max_seqlen_q > 1) {
      const int sp = hip_status(vox::launch_prefill(a, max_seqlen_q, s), "prefill_attn launch");
      if (sp != VOX_OK) return sp;
    }
    return launch_decode_slices(d, batch, num_kv_heads, plan, workspace, s);
  }
  return hip_status(vox::launch_prefill(a, max_seqlen_q, s), "prefill_attn launch");
}

int vox_prefill_attn_store(const void* q, int64_t q_row_stride, const void* key, const void* value,
                           int64_t key_row_stride, int64_t value_row_stride, const int32_t* slot_mapping,
                           void* k_cache, void* v_cache, int64_t num_slots, int64_t num_tokens,
                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch, int max_seqlen_q,
                           int num_heads, int num_kv_heads, int head_dim, float softmax_scale, int causal, void* out,
                           int64_t out_row_stride, void* stream) {
  if (batch < 0 || max_seqlen_q < 0 || num_tokens < 0)
    return fail(VOX_EINVAL, "prefill_attn_store: negative batch, max_seqlen_q or num_tokens");
  if (!key || !value || !k_cache || !v_cache || !slot_mapping || !cu_seqlens_q || !cu_seqlens_k)
    return fail(VOX_EINVAL, "prefill_attn_store: null pointer argument");
  if (num_slots <= 0) return fail(VOX_EINVAL, "prefill_attn_store: empty cache");
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (num_kv_heads <= 0 || head_dim <= 0 || key_row_stride < row || value_row_stride < row)
    return fail(VOX_EINVAL, "prefill_attn_store: key / value row strides smaller than num_kv_heads * head_dim");
  // every argument is checked before anything is launched
  const bool attend = batch > 0 && max_seqlen_q > 0;
  vox::PrefillArgs a;
  if (attend) {
    if (!out) return fail(VOX_EINVAL, "prefill_attn_store: null out");
    if (out_row_stride < (int64_t)num_heads * head_dim || out_row_stride % 4 || ((uintptr_t)out & 7u))
      return fail(VOX_EINVAL, "prefill_attn_store: bad out row stride or alignment");
    const int st = prefill_setup("prefill_attn_store", q, q_row_stride, key, value, key_row_stride,
                                 value_row_stride, nullptr, nullptr, 0, 0, nullptr, 0, 0, cu_seqlens_q, cu_seqlens_k,
                                 batch, max_seqlen_q, 0, 0, num_heads, num_kv_heads, head_dim, softmax_scale, causal,
                                 &a);
    if (st != VOX_OK) return st;
  }
  const bool vec16 = row % 8 == 0 && key_row_stride % 8 == 0 && value_row_stride % 8 == 0 && aligned16(key) &&
                     aligned16(value) && aligned16(k_cache) && aligned16(v_cache);
  if (!attend || !vec16 || num_tokens == 0) {
    // no launch to ride in, nothing to store, or rows the 16-byte copy cannot move: the two calls
    const int st = vox_store_kvcache(key, value, key_row_stride, value_row_stride, k_cache, v_cache, num_slots,
                                     slot_mapping, num_tokens, num_kv_heads, head_dim, stream);
    if (st != VOX_OK || !attend) return st;
    return vox_prefill_attn(q, q_row_stride, key, value, key_row_stride, value_row_stride, nullptr, nullptr, 0, 0,
                            nullptr, 0, 0, cu_seqlens_q, cu_seqlens_k, batch, max_seqlen_q, 0, 0, num_heads,
                            num_kv_heads, head_dim, softmax_scale, causal, out, out_row_stride, VOX_PLAN_NONE,
                            nullptr, 0, stream);
  }
  a.out = (uint16_t*)out;
  a.out_row_stride = out_row_stride;
  a.store_slots = slot_mapping;
  a.store_k_cache = (uint16_t*)k_cache;
  a.store_v_cache = (uint16_t*)v_cache;
  a.store_rows = num_tokens;
  a.store_num_slots = num_slots;
  return hip_status(vox::launch_prefill(a, max_seqlen_q, (hipStream_t)stream), "prefill_attn_store launch");
}

int vox_prefill_attn_store_paged(const void* q, int64_t q_row_stride, const void* key, const void* value,
                                 int64_t key_row_stride, int64_t value_row_stride, const int32_t* slot_mapping,
                                 int64_t num_tokens, void* k_cache, void* v_cache, int64_t num_blocks, int block_size,
                                 const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                                 const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch, int max_seqlen_q,
                                 int num_heads, int num_kv_heads, int head_dim, float softmax_scale, int causal,
                                 void* out, int64_t out_row_stride, int plan, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  if (batch < 0 || max_seqlen_q < 0 || num_tokens < 0)
    return fail(VOX_EINVAL, "prefill_attn_store_paged: negative batch, max_seqlen_q or num_tokens");
  if (!key || !value || !k_cache || !v_cache || !slot_mapping || !block_tables || !cu_seqlens_q || !cu_seqlens_k)
    return fail(VOX_EINVAL, "prefill_attn_store_paged: null pointer argument");
  if (num_blocks <= 0 || block_size <= 0) return fail(VOX_EINVAL, "prefill_attn_store_paged: empty cache");
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (num_kv_heads <= 0 || head_dim <= 0 || key_row_stride < row || value_row_stride < row)
    return fail(VOX_EINVAL, "prefill_attn_store_paged: key / value row strides smaller than num_kv_heads * head_dim");
  // every argument is checked before anything is launched
  const bool attend = batch > 0 && max_seqlen_q > 0;
  vox::PrefillArgs a;
  if (attend) {
    if (!out) return fail(VOX_EINVAL, "prefill_attn_store_paged: null out");
    if (out_row_stride < (int64_t)num_heads * head_dim || out_row_stride % 4 || ((uintptr_t)out & 7u))
      return fail(VOX_EINVAL, "prefill_attn_store_paged: bad out row stride or alignment");
    const int st = prefill_setup("prefill_attn_store_paged", q, q_row_stride, key, value, key_row_stride,
                                 value_row_stride, k_cache, v_cache, num_blocks, block_size, block_tables, bt_stride,
                                 max_blocks, cu_seqlens_q, cu_seqlens_k, batch, max_seqlen_q, 0, 0, num_heads,
                                 num_kv_heads, head_dim, softmax_scale, causal, &a);
    if (st != VOX_OK) return st;
    a.out = (uint16_t*)out;
    a.out_row_stride = out_row_stride;
    if (varlen_decode_rows(a, workspace, num_kv_heads)) {
      const int sw = check_varlen_workspace("prefill_attn_store_paged", batch, plan, workspace, workspace_bytes);
      if (sw != VOX_OK) return sw;
    }
  }
  if (plan != VOX_PLAN_NONE && plan != VOX_PLAN_RECORD && plan != VOX_PLAN_REUSE)
    return fail(VOX_EINVAL, "prefill_attn_store_paged: plan mode %d", plan);
  // The store rides in the attention launch: in a mixed launch both roles read each sequence's new keys from the rows
  // (by position) and the merge kernel's extra workgroups write the rows into the caches after every read. Else the
  // two calls.
  const bool vec16 = row % 8 == 0 && key_row_stride % 8 == 0 && value_row_stride % 8 == 0 && aligned16(key) &&
                     aligned16(value) && aligned16(k_cache) && aligned16(v_cache) &&
                     key_row_stride < (1 << 24) && value_row_stride < (1 << 24);
  const bool decode_rows = attend && varlen_decode_rows(a, workspace, num_kv_heads);
  const bool fold_mixed = attend && num_tokens > 0 && max_seqlen_q > 1 && vec16 && decode_rows &&
                          vox::mixed_launch_fits(a, num_kv_heads);
  // without the decode rows' workspace the prefill kernel takes every row: the store rides in its launch as in the
  // packed form (the last workgroups copy the rows), the new keys read from the rows
  const bool fold_plain = attend && num_tokens > 0 && vec16 && !decode_rows && block_size % 64 == 0;
  if (fold_plain) {
    a.k_src = (const uint16_t*)key;
    a.v_src = (const uint16_t*)value;
    a.k_row_stride = key_row_stride;
    a.v_row_stride = value_row_stride;
    a.new_from_rows = 1;
    a.store_slots = slot_mapping;
    a.store_k_cache = (uint16_t*)k_cache;
    a.store_v_cache = (uint16_t*)v_cache;
    a.store_rows = num_tokens;
    a.store_num_slots = num_blocks * block_size;
    return hip_status(vox::launch_prefill(a, max_seqlen_q, (hipStream_t)stream), "prefill_attn_store_paged launch");
  }
  if (!fold_mixed) {
    const int st = vox_store_kvcache(key, value, key_row_stride, value_row_stride, k_cache, v_cache,
                                     num_blocks * block_size, slot_mapping, num_tokens, num_kv_heads, head_dim, stream);
    if (st != VOX_OK || !attend) return st;
    return vox_prefill_attn(q, q_row_stride, key, value, key_row_stride, value_row_stride, k_cache, v_cache, num_blocks,
                            block_size, block_tables, bt_stride, max_blocks, cu_seqlens_q, cu_seqlens_k, batch,
                            max_seqlen_q, 0, 0, num_heads, num_kv_heads, head_dim, softmax_scale, causal, out,
                            out_row_stride, plan, workspace, workspace_bytes, stream);
  }
  a.skip_single = 1;
  a.persistent = 1;
  a.k_src = (const uint16_t*)key;
  a.v_src = (const uint16_t*)value;
  a.k_row_stride = key_row_stride;
  a.v_row_stride = value_row_stride;
  a.new_from_rows = 1;
  vox::DecodeArgs d = varlen_decode_args(a, q_row_stride, num_blocks, num_heads, num_kv_heads);
  d.slot_mapping = slot_mapping;
  d.new_k = (const uint16_t*)key;
  d.new_v = (const uint16_t*)value;
  d.new_k_stride = key_row_stride;
  d.new_v_stride = value_row_stride;
  d.copy_rows = num_tokens;
  // about one batch of 16-byte copies per thread of a 256-thread workgroup (16 rows of 2 x 256 bf16), at most 256
  const int64_t per_wg = 4 * 256 / (2 * row / 8);
  const int64_t cw = (num_tokens + per_wg - 1) / per_wg;
  d.copy_wgs = (int)(cw < 256 ? cw : 256);
  const vox::DecodeArgs dw = with_workspace(d, batch, plan, workspace);
  return hip_status(vox::launch_mixed(a, max_seqlen_q, dw, num_kv_heads, (hipStream_t)stream),
                    "prefill_attn_store_paged mixed launch");
}

}  // extern "C"

namespace {
// A KV store riding in an int8 prefill launch (vox_prefill_attn_int8_store): rows [0, rows) of the key / value rows
// to slot_mapping's slots
struct RidingStore {
  const int32_t* slot_mapping;
  void* k_cache;
  void* v_cache;
  int64_t num_slots;
  int64_t rows;
  bool paged;  // paged tiles: the launch reads each sequence's new keys from the rows
};

int prefill_int8(const char* fn, const void* q, int64_t q_row_stride, const void* key, const void* value,
                 int64_t key_row_stride, int64_t value_row_stride, const void* k_cache, const void* v_cache,
                 int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                 const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch, int max_seqlen_q,
                 int uniform_seqlen_q, int uniform_seqlen_k, int num_heads, int num_kv_heads, int head_dim,
                 float softmax_scale, int causal, const float* inv_smooth, void* out_q, int64_t out_q_row_stride,
                 float* out_scale, int64_t num_tokens, void* workspace, size_t workspace_bytes,
                 const RidingStore* store, bool launch, hipStream_t stream) {
  if (!out_q || !out_scale) return fail(VOX_EINVAL, "%s: null out_q or out_scale", fn);
  if (num_kv_heads != 1 && num_kv_heads != 2)
    return fail(VOX_EINVAL, "%s: num_kv_heads %d unsupported (1 or 2)", fn, num_kv_heads);
  if (out_q_row_stride < (int64_t)num_heads * head_dim || out_q_row_stride % 4 || ((uintptr_t)out_q & 3u))
    return fail(VOX_EINVAL, "%s: bad out_q row stride or alignment", fn);
  if (((uintptr_t)out_scale & 3u) || (inv_smooth && !aligned16(inv_smooth)))
    return fail(VOX_EINVAL, "%s: out_scale must be 4-byte and inv_smooth 16-byte aligned", fn);
  vox::PrefillArgs a;
  const int st = prefill_setup(fn, q, q_row_stride, key, value, key_row_stride, value_row_stride, k_cache, v_cache,
                               num_blocks, block_size, block_tables, bt_stride, max_blocks, cu_seqlens_q,
                               cu_seqlens_k, batch, max_seqlen_q, uniform_seqlen_q, uniform_seqlen_k, num_heads,
                               num_kv_heads, head_dim, softmax_scale, causal, &a);
  if (st != VOX_OK) return st;
  if (!cu_seqlens_q && num_tokens != (int64_t)batch * uniform_seqlen_q)
    return fail(VOX_EINVAL, "%s: num_tokens %lld != batch x uniform_seqlen_q", fn, (long long)num_tokens);
  // rows at or past num_tokens are never read or written, whatever cu_seqlens_q (device memory the host cannot
  // check here) says: the outputs and the two-pass scratch are sized by num_tokens
  a.row_limit = num_tokens;
  const size_t need = workspace ? vox_prefill_int8_workspace_bytes(num_tokens, batch, max_seqlen_q, num_heads,
                                                                   num_kv_heads, head_dim, causal)
                                : 0;
  if (need && (workspace_bytes < need || !aligned16(workspace)))
    return fail(VOX_EINVAL, "%s: workspace of %zu bytes (16-byte aligned), %zu needed", fn, workspace_bytes, need);
  if (!launch) return VOX_OK;  // (arguments checked only)
  if (store) {
    if (store->paged) {
      a.k_src = (const uint16_t*)key;
      a.v_src = (const uint16_t*)value;
      a.k_row_stride = key_row_stride;
      a.v_row_stride = value_row_stride;
      a.new_from_rows = 1;
    }
    a.store_slots = store->slot_mapping;
    a.store_k_cache = (uint16_t*)store->k_cache;
    a.store_v_cache = (uint16_t*)store->v_cache;
    a.store_rows = store->rows;
    a.store_num_slots = store->num_slots;
  }
  if (need) {
    // two passes: the bf16 kernel into the workspace ([T, H * 128] bf16; a riding store copied in that launch), then
    // the per-token quantization
    a.out = (uint16_t*)workspace;
    a.out_row_stride = (int64_t)num_heads * head_dim;
    const int st1 = hip_status(vox::launch_prefill(a, max_seqlen_q, stream), "prefill_attn_int8 launch");
    if (st1 != VOX_OK) return st1;
    return hip_status(vox::launch_quantize_rows((const uint16_t*)workspace, num_tokens, num_heads * head_dim,
                                                inv_smooth, (int8_t*)out_q, out_q_row_stride, out_scale, stream),
                      "prefill_attn_int8 quantization launch");
  }
  a.inv_smooth = inv_smooth;
  a.out_q = (int8_t*)out_q;
  a.out_row_stride = out_q_row_stride;
  a.out_scale = out_scale;
  return hip_status(vox::launch_prefill_int8(a, max_seqlen_q, stream), "prefill_attn_int8 launch");
}
}  // namespace

extern "C" {

int vox_prefill_attn_int8(const void* q, int64_t q_row_stride, const void* key, const void* value,
                          int64_t key_row_stride, int64_t value_row_stride, const void* k_cache, const void* v_cache,
                          int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                          int max_blocks, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch,
                          int max_seqlen_q, int uniform_seqlen_q, int uniform_seqlen_k, int num_heads,
                          int num_kv_heads, int head_dim, float softmax_scale, int causal, const float* inv_smooth,
                          void* out_q, int64_t out_q_row_stride, float* out_scale, int64_t num_tokens,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 0 || max_seqlen_q < 0 || num_tokens < 0)
    return fail(VOX_EINVAL, "prefill_attn_int8: negative batch, max_seqlen_q or num_tokens");
  if (batch == 0 || max_seqlen_q == 0 || num_tokens == 0) return VOX_OK;
  return prefill_int8("prefill_attn_int8", q, q_row_stride, key, value, key_row_stride, value_row_stride, k_cache,
                      v_cache, num_blocks, block_size, block_tables, bt_stride, max_blocks, cu_seqlens_q,
                      cu_seqlens_k, batch, max_seqlen_q, uniform_seqlen_q, uniform_seqlen_k, num_heads, num_kv_heads,
                      head_dim, softmax_scale, causal, inv_smooth, out_q, out_q_row_stride, out_scale, num_tokens,
                      workspace, workspace_bytes, nullptr, true, (hipStream_t)stream);
}

int vox_prefill_attn_int8_store(const void* q, int64_t q_row_stride, const void* key, const void* value,
                                int64_t key_row_stride, int64_t value_row_stride, const int32_t* slot_mapping,
                                int64_t store_rows, void* k_cache, void* v_cache, int64_t num_blocks, int block_size,
                                const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch, int max_seqlen_q,
                                int num_heads, int num_kv_heads, int head_dim, float softmax_scale, int causal,
                                const float* inv_smooth, void* out_q, int64_t out_q_row_stride, float* out_scale,
                                int64_t num_tokens, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "prefill_attn_int8_store";
  if (batch < 0 || max_seqlen_q < 0 || num_tokens < 0 || store_rows < 0)
    return fail(VOX_EINVAL, "%s: negative batch, max_seqlen_q, num_tokens or store_rows", fn);
  if (!key || !value || !k_cache || !v_cache || !slot_mapping || !cu_seqlens_q || !cu_seqlens_k)
    return fail(VOX_EINVAL, "%s: null pointer argument", fn);
  if (num_blocks <= 0 || block_size <= 0) return fail(VOX_EINVAL, "%s: empty cache", fn);
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (num_kv_heads <= 0 || head_dim <= 0 || key_row_stride < row || value_row_stride < row)
    return fail(VOX_EINVAL, "%s: key / value row strides smaller than num_kv_heads * head_dim", fn);
  // every argument is checked before anything is launched
  const bool paged = block_tables != nullptr;
  const bool attend = batch > 0 && max_seqlen_q > 0 && num_tokens > 0;
  const void* kc_read = paged ? k_cache : nullptr;
  const void* vc_read = paged ? v_cache : nullptr;
  if (attend) {
    const int st = prefill_int8(fn, q, q_row_stride, key, value, key_row_stride, value_row_stride, kc_read, vc_read,
                                num_blocks, block_size, block_tables, bt_stride, max_blocks, cu_seqlens_q,
                                cu_seqlens_k, batch, max_seqlen_q, 0, 0, num_heads, num_kv_heads, head_dim,
                                softmax_scale, causal, inv_smooth, out_q, out_q_row_stride, out_scale, num_tokens,
                                workspace, workspace_bytes, nullptr, false, nullptr);
    if (st != VOX_OK) return st;
  }
  // the store rides in the launch over packed keys, or over paged tiles that read the new keys from the rows
  const bool vec16 = row % 8 == 0 && key_row_stride % 8 == 0 && value_row_stride % 8 == 0 && aligned16(key) &&
                     aligned16(value) && aligned16(k_cache) && aligned16(v_cache) && key_row_stride < (1 << 24) &&
                     value_row_stride < (1 << 24);
  if (!attend || !vec16 || store_rows == 0 || (paged && block_size % 64 != 0)) {
    // no launch to ride in, nothing to store, or rows / blocks the riding copy does not take: the two calls
    const int st = vox_store_kvcache(key, value, key_row_stride, value_row_stride, k_cache, v_cache,
                                     num_blocks * block_size, slot_mapping, store_rows, num_kv_heads, head_dim, stream);
    if (st != VOX_OK || !attend) return st;
    return vox_prefill_attn_int8(q, q_row_stride, key, value, key_row_stride, value_row_stride, kc_read, vc_read,
                                 num_blocks, block_size, block_tables, bt_stride, max_blocks, cu_seqlens_q,
                                 cu_seqlens_k, batch, max_seqlen_q, 0, 0, num_heads, num_kv_heads, head_dim,
                                 softmax_scale, causal, inv_smooth, out_q, out_q_row_stride, out_scale, num_tokens,
                                 workspace, workspace_bytes, stream);
  }
  const RidingStore rs{slot_mapping, k_cache, v_cache, num_blocks * block_size, store_rows, paged};
  return prefill_int8(fn, q, q_row_stride, key, value, key_row_stride, value_row_stride, kc_read, vc_read, num_blocks,
                      block_size, block_tables, bt_stride, max_blocks, cu_seqlens_q, cu_seqlens_k, batch, max_seqlen_q,
                      0, 0, num_heads, num_kv_heads, head_dim, softmax_scale, causal, inv_smooth, out_q,
                      out_q_row_stride, out_scale, num_tokens, workspace, workspace_bytes, &rs, true,
                      (hipStream_t)stream);
}

size_t vox_prefill_int8_workspace_bytes(int64_t num_tokens, int batch, int max_seqlen_q, int num_heads,
                                        int num_kv_heads, int head_dim, int causal) {
  if (num_tokens <= 0 || head_dim != kHeadDim || num_heads <= 0 || num_heads * head_dim > 2048) return 0;
  if (!vox::prefill_int8_two_pass(batch, max_seqlen_q, num_heads, num_kv_heads, causal)) return 0;
  return (size_t)num_tokens * num_heads * head_dim * 2;
}

int vox_copy_kv_block_prefix(void* kv, int64_t num_planes, int64_t num_blocks, int block_size,
                              int64_t per_token, int elem_bytes, const int32_t* entries, int num_entries,
                              int max_tokens, void* stream) {
  if (num_entries < 0 || num_planes < 0) return fail(VOX_EINVAL, "copy_kv_block_prefix: negative count");
  if (num_entries == 0 || num_planes == 0 || max_tokens <= 0) return VOX_OK;
  if (!kv || !entries) return fail(VOX_EINVAL, "copy_kv_block_prefix: null kv or entries");
  if (elem_bytes != 2) return fail(VOX_EINVAL, "copy_kv_block_prefix: %d-byte elements unsupported (2 only)", elem_bytes);
  if (num_blocks <= 0 || block_size <= 0 || per_token <= 0)
    return fail(VOX_EINVAL, "copy_kv_block_prefix: bad cache shape");
  if (num_planes > 65535) return fail(VOX_EINVAL, "copy_kv_block_prefix: more than 65535 planes");
  if (max_tokens > block_size) max_tokens = block_size;
  vox::CopyArgs a;
  a.kv = kv;
  a.num_planes = num_planes;
  a.num_blocks = num_blocks;
  a.block_size = block_size;
  a.per_token = per_token;
  a.entries = entries;
  a.num_entries = num_entries;
  const bool vec16 = per_token % 8 == 0 && aligned16(kv);
  return hip_status(vox::launch_copy_block_prefix(a, max_tokens, vec16, (hipStream_t)stream),
                    "copy_kv_block_prefix launch");
}

}  // extern "C"
