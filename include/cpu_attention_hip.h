/*
 * cpu_attention_hip.h -- the C ABI of the gfx950 (MI355X) build of cpu-attention's
 * three ops: reshape_and_cache, paged decode (flash_attn_with_kvcache) and dense
 * prefill (flash_attn_func).
 *
 * Every entry takes plain device pointers, element counts and element strides (no
 * torch types), validates what it can see without reading device memory, enqueues
 * its kernels on `stream` (a hipStream_t; NULL = the legacy default stream) and
 * returns without synchronising.
 *
 * Return codes:
 *   CA_OK (0)        the kernels were enqueued;
 *   CA_DECLINED (1)  the arguments are outside what the kernels take (shape,
 *                    dtype, head_dim, page size, alignment, workspace): nothing
 *                    was enqueued.  The Python layer turns this into the
 *                    reference's ValueError / NotImplementedError, or copies the
 *                    operands to a readable layout and calls again;
 *   CA_HIP_ERROR (<0) a HIP launch error; ca_status_string() names it.
 *
 * The entries are re-entrant and keep no global mutable state (ca_decode_noalloc
 * aside: it uses one fixed scratch buffer per GPU).  None allocates: outputs and
 * split-K scratch are passed in by the caller.
 *
 * Data-dependent bounds (a slot past the cache's end, a length beyond the page
 * table's capacity, a page-table entry that names no block) are guarded inside
 * the kernels: such a token is not stored, such a position is not read.  The
 * reference raises ValueError for the first two; the Python layer does that
 * check on the host before calling (see cpu_attention/_kernel.py).
 *
 * Cache layout (the reference's PageLayout, cpu_attention/_mojo/src/paged_attn.mojo:58-130,
 * x86 mapping): k_cache and v_cache are [num_blocks, num_heads, page_size, head_dim],
 * contiguous.  Block (b, h) starts at element (b*H + h)*P*E.  Within it:
 *   fp32 K: element K[d][t]  at  d*P + t;
 *   bf16 K: 32-bit words [E/2][P]; word (d2, t) holds the bf16 pair
 *           (K[2*d2], K[2*d2+1]), i.e. element (d2*P + t)*2 + (d & 1);
 *   V (both dtypes): rows [P][E], element t*E + d.
 */
#ifndef CPU_ATTENTION_HIP_H
#define CPU_ATTENTION_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CA_ABI_VERSION 3

enum { CA_F32 = 0, CA_BF16 = 1 };

/* CA_SCRATCH_EXCEEDED: ca_decode_noalloc only -- the call needs more split-K
 * scratch than the library's fixed buffer holds; nothing was enqueued. */
enum { CA_OK = 0, CA_DECLINED = 1, CA_SCRATCH_EXCEEDED = 2, CA_HIP_ERROR = -1 };

/* reshape_and_cache (cpu_attention/cache.py:13-25, native entry `store`
 * cpu_attention/_mojo/src/_C.mojo:174-213).  Token i of key/value
 * [num_tokens, num_heads, head_dim] (heads and dims contiguous, any token
 * stride, the same for both) goes to slot s = slot_mapping[i]: block s / P,
 * position s % P.  s < 0 skips the token; s >= num_blocks*P is not stored. */
typedef struct ca_store_args {
  const void* key;
  const void* value;
  int64_t token_stride;  /* elements between consecutive tokens of key/value
                            (not read when num_tokens == 1) */
  void* k_cache;
  void* v_cache;
  const int64_t* slot_mapping;  /* [num_tokens], int64 */
  int64_t num_tokens;
  int64_t num_heads;
  int64_t head_dim;   /* 32, 64 or 128 */
  int64_t page_size;  /* a positive multiple of 16 */
  int64_t num_blocks;
  int32_t dtype;      /* CA_F32 or CA_BF16 */
  int32_t reserved;
} ca_store_args;

int ca_store(const ca_store_args* args, void* stream);

/* Paged decode (flash_attn_interface.py:37-127, native entry `decode`
 * _C.mojo:87-171): one query row per (sequence, head) against the sequence's
 * cached K/V, online softmax in base 2, fp32 accumulation, output in the input
 * dtype; a row with no key is exactly 0.
 *
 * With k_new/v_new the new tokens are stored first:
 *   slots == NULL: new_tokens tokens per sequence (0 counts as 1), token j of
 *                  sequence s at position lens[s] + j through page_table (lens is
 *                  the length before the store; the row attends lens[s] +
 *                  new_tokens keys; lens[s] < 0 stores nothing, positions past
 *                  the page table are not stored).  One token is the reference's
 *                  append; several are its prompt append, which the reference
 *                  builds from slot arithmetic and reshape_and_cache
 *                  (flash_attn_interface.py:109-117) and this entry computes
 *                  inside the store kernel;
 *   slots != NULL: one token per sequence at slot slots[s] (negative skips), and
 *                  lens[s] is the length after the store (the engine path,
 *                  examples/ops.py:19-25); new_tokens must be 0 or 1.
 * Without k_new/v_new the row attends lens[s] keys.
 *
 * q: [num_seqs, num_heads, head_dim] rows, heads and dims contiguous, sequence
 * stride q_stride (elements).  k_new, v_new: rows of [num_seqs * new_tokens,
 * num_heads, head_dim] (token j of sequence s is row s * new_tokens + j), heads
 * and dims contiguous, row stride kv_stride.
 * out: [num_seqs, num_heads, head_dim] contiguous.
 * workspace: at least ca_decode_workspace_bytes(...) bytes of device memory,
 * 256-byte aligned; its contents need not be initialised. */
typedef struct ca_decode_args {
  const void* q;
  int64_t q_stride;
  void* k_cache;
  void* v_cache;
  const void* k_new;   /* NULL: no store */
  const void* v_new;
  int64_t kv_stride;
  const int64_t* slots;      /* NULL or [num_seqs] int64 */
  const int32_t* lens;       /* [num_seqs] int32 */
  const int32_t* page_table; /* [num_seqs, page_table_width] int32, contiguous */
  int64_t page_table_width;
  void* out;
  int64_t num_seqs;
  int64_t num_heads;
  int64_t head_dim;
  int64_t page_size;
  int64_t num_blocks;
  float scale;        /* softmax scale (the caller resolves the 1/sqrt(E) default) */
  int32_t dtype;
  void* workspace;
  int64_t workspace_bytes;
  int64_t new_tokens;  /* tokens per sequence in k_new/v_new (0 or 1: one) */
} ca_decode_args;

/* ca_decode_workspace_bytes: the split-K scratch a call of these shapes needs
 * with its preferred tile size, for the larger of a bf16 and an fp32 call (the
 * tile size depends on the element size too: 256-key tiles only for rows of at
 * most 128 bytes).  0: none; rows whose page table holds at most one block of
 * tiles, 512 keys with 64-key tiles or 2048 with 256-key tiles, need none.
 * Otherwise the rows' block partials, and for calls of 64 to 512 rows whose page
 * table holds at most 4 blocks of tiles (whose partials the row's last block
 * merges inside the decode kernel) one 8-byte counter per row, tagged per call,
 * so that no clearing is needed; calls that overlap must not share a workspace.
 * It is not monotonic in num_seqs: the preferred tile size depends on the
 * number of rows.  ca_decode therefore takes 256-key tiles when the workspace it
 * is given is too small for the preferred ones but holds those; with one tile
 * size the need grows with the rows, so a workspace sized once for the largest
 * batch of a page table serves every smaller batch (its output may then differ
 * from the preferred tiles' in the last bits, within the same tolerance). */
int64_t ca_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads, int64_t head_dim,
                                  int64_t page_size, int64_t page_table_width);
int ca_decode(const ca_decode_args* args, void* stream);

/* ca_decode without a workspace argument and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory at call time (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as ca_decode;
 * args->workspace and args->workspace_bytes are ignored.  The split-K scratch
 * is a fixed device array, CA_DECODE_NOALLOC_SCRATCH_BYTES (32 MiB) per GPU, in
 * a code object of its own that HIP loads on a device at the first
 * ca_decode_noalloc call there that needs scratch (processes that never call it
 * do not reserve it); it is then held until the process ends.  Its address is
 * resolved once per device (the current device at the call; `stream` must
 * belong to it).  A call whose ca_decode_workspace_bytes(...) exceeds that size
 * runs with 256-key tiles (fewer partials per row; its output may then differ
 * from ca_decode's in the last bits, within the same tolerance); if those still
 * do not fit, it returns CA_SCRATCH_EXCEEDED and enqueues nothing (32 MiB
 * covers, e.g., 4096 rows of E=128 up to 30,720 keys of page-table capacity).
 * Rows whose page table holds at most one block of tiles (512 keys with 64-key
 * tiles, 2048 with 256-key tiles) need no scratch.  Every call on a GPU that
 * uses the scratch shares that GPU's one buffer, so the entry orders such calls
 * itself: each one's kernels wait, on its stream, for an event recorded after
 * the previous such call's kernels on that GPU (whichever stream they ran on),
 * and host threads take turns for the wait-launch-record sequence (one event per
 * GPU, created at the same set-up as the address lookup).  A stream under graph
 * capture neither waits nor records: calls captured into graphs, and the graphs'
 * replays, must be ordered by the caller against every other use of the buffer.
 * The buffer needs no clearing: each call writes every partial it reads before
 * reading it. */
#define CA_DECODE_NOALLOC_SCRATCH_BYTES (32ll << 20)
int ca_decode_noalloc(const ca_decode_args* args, void* stream);

/* Dense prefill (flash_attn_interface.py:168-193, native entry `flash`
 * _C.mojo:232-316).  q [batch, seq_q, H, E], k/v [batch, seq_k, H, E] with any
 * batch/token/head strides (elements; the head_dim stride is 1).  Causal is
 * bottom-right aligned: query i sees keys j <= i + seq_k - seq_q; a row that sees
 * no key is exactly 0.  out is a contiguous [batch, seq_q, H, E] in the input
 * dtype.  Calls whose keys are split over several blocks leave partials in the
 * workspace: few-row calls (seq_q <= 4 bf16; <= 8 fp32, or <= 16 with batch x
 * heads >= 256), and calls with fewer
 * than 256 query blocks of 256 rows (bf16) or 512 of 128 rows (fp32) over long
 * key ranges (bf16 calls with fewer than twice as many keys as rows only below
 * 64 query blocks, below 128 over 2048 keys or more, or at 128 over 4096 or
 * more; under 1024 keys only non-causal calls below 16 query blocks).
 * Pass at least the bytes ca_flash_workspace_bytes() asks for (0 means none is
 * needed; it answers for the larger of the causal and non-causal call; a
 * shorter workspace declines the call), 16-byte aligned (256 recommended; a
 * misaligned one declines a call that uses it); its contents need not be
 * initialised.  The
 * reference's entry grows its workspace on request the same way
 * (flash_attn_interface.py:186-193). */
typedef struct ca_flash_args {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t batch;
  int64_t seq_q;
  int64_t seq_k;
  int64_t num_heads;
  int64_t head_dim;
  int64_t q_strides[3];  /* batch, token, head */
  int64_t k_strides[3];
  int64_t v_strides[3];
  float scale;
  int32_t causal;
  int32_t dtype;
  int32_t reserved;
  void* workspace;
  int64_t workspace_bytes;
} ca_flash_args;

int64_t ca_flash_workspace_bytes(int64_t batch, int64_t seq_q, int64_t seq_k,
                                 int64_t num_heads, int64_t head_dim, int32_t dtype);
int ca_flash(const ca_flash_args* args, void* stream);

/* ABI version (CA_ABI_VERSION), a build description, and a readable status. */
int ca_abi_version(void);
const char* ca_version(void);
const char* ca_status_string(int status);

#ifdef __cplusplus
}
#endif

#endif /* CPU_ATTENTION_HIP_H */
