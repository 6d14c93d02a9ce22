/*
 * vk_gemm.h -- C ABI of the MI355X (gfx950) GEMM kernel suite.
 *
 * One shared library, libvk_gemm.so, built from vibekernel_amd/csrc/ with
 * hipcc --offload-arch=gfx950.  Plain C types only: no HIP, torch or C++
 * types cross this boundary (a stream is passed as void*, NULL = the null
 * stream of the current device).
 *
 * Reference interface replaced (paths relative to the reference repository):
 *   results/naive_cycle4/include/playground/matmul.hpp:11-13
 *     template <typename DType, uint8_t Version>
 *     void matmul(size_t m, size_t n, size_t k, const DType* A, const DType* B, DType* C);
 *   specialised per version by PLAYGROUND_MATMUL_DEC (matmul.hpp:16-19) and
 *   called through PLAYGOUND_MATMUL_CALL (matmul.hpp:21-23) from
 *   results/ralph_loop_fable/src/main.cpp:38-41.
 *
 * Semantics kept from the reference:
 *   C = A . B, all three row-major and dense (lda = k, ldb = n, ldc = n),
 *   alpha = 1, beta = 0: C is fully overwritten and never read
 *   (matmul_f16_v0_cblas.cpp:22-23).  A, B, C are DEVICE pointers for every
 *   version >= 1 (main.cpp:49-51).  The launch is asynchronous on the stream;
 *   nothing inside synchronises.  fp16 inputs are accumulated in fp32.
 *
 * Differences (the reference returns void and has no error channel):
 *   every entry point returns VK_OK or a negative vk_status and never exits;
 *   the output dtype may be fp32 as well as the input dtype;
 *   the stream is explicit; version 0 (the CPU cBLAS ground truth) is not in
 *   this library -- it lives with the task1 harness, as in the reference.
 */
#ifndef VK_GEMM_H
#define VK_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VK_GEMM_ABI_VERSION 1

typedef enum vk_dtype {
  VK_DTYPE_F16 = 1, /* IEEE binary16 ("float16_t" = half in the reference, system.hpp:29) */
  VK_DTYPE_F32 = 2, /* IEEE binary32 ("float32_t", system.hpp:27) */
  /* Not dtypes: they make every int value a valid vk_dtype, so a bad value
   * from a C caller is reported (VK_ERR_DTYPE / VK_ERR_VERSION) rather than
   * being undefined behaviour in the C++ library. */
  VK_DTYPE_INT_MIN_ = -2147483647 - 1,
  VK_DTYPE_INT_MAX_ = 2147483647
} vk_dtype;

typedef enum vk_status {
  VK_OK = 0,
  VK_ERR_VERSION = -1,   /* no such version for this input dtype */
  VK_ERR_DTYPE = -2,     /* unsupported (input, output) dtype pair */
  VK_ERR_SHAPE = -3,     /* shape not handled by this version (see vk_caps) */
  VK_ERR_ALIGN = -4,     /* a pointer is not aligned as this version needs */
  VK_ERR_NULL = -5,      /* NULL operand with a non-empty shape */
  VK_ERR_WORKSPACE = -6, /* caller workspace smaller than vk_gemm_workspace_bytes() */
  VK_ERR_HIP = -7,       /* HIP runtime error (launch, allocation, device query) */
  VK_ERR_RANGE = -8      /* a dimension exceeds what the version indexes (2^31-1) */
} vk_status;

/* What a version handles.  A shape is accepted when m % div_m == 0,
 * n % div_n == 0, k % div_k == 0, m <= max_m, and the operands are aligned to
 * align_bytes.  tolerance_tier: 0 = fp32 accumulation in one pass (the
 * reference's strict tier, mean relative error ~3e-5 on N(0,1) data);
 * 1 = relaxed (partials rounded below fp32). */
typedef struct vk_caps {
  int version;
  int in_dtype;
  int out_dtype_mask; /* bit (1 << vk_dtype) set for each supported output */
  uint32_t div_m, div_n, div_k;
  uint64_t max_m;
  uint32_t align_bytes;
  uint32_t tile_m, tile_n, tile_k; /* workgroup macro tile */
  uint32_t threads;                /* threads per workgroup */
  uint32_t lds_bytes;              /* LDS per workgroup */
  int tolerance_tier;
  int uses_workspace;
} vk_caps;

/* C = A . B on `stream`.  Library-managed workspace: a version that needs one
 * allocates it on its first call on a device (like the reference's
 * function-local statics, matmul_f16_v42_shfl2.cu:496-519) and keeps it until
 * vk_gemm_release() or process exit.  All calls of such versions on one
 * device share that workspace, so they must not run concurrently (issue them
 * on one stream, or order them); concurrent callers pass their own
 * workspaces to vk_gemm_ws.  Under stream capture a call that would use the
 * library workspace returns VK_ERR_WORKSPACE (a captured graph would keep an
 * address that a later call may free); capture such calls with vk_gemm_ws.
 * Calls that need no workspace may be captured. */
int vk_gemm(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n, size_t k,
            const void* A, const void* B, void* C, void* stream);

/* Same, with a caller-owned device workspace of at least
 * vk_gemm_workspace_bytes() bytes (may be NULL when that is 0).  Never
 * allocates.  Safe under stream capture: the counters the kernels share are
 * cleared by a small kernel (not a memset) in every call, so each replay of a
 * captured graph starts from zero; calls sharing one workspace must not
 * overlap. */
int vk_gemm_ws(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n, size_t k,
               const void* A, const void* B, void* C, void* workspace, size_t workspace_bytes,
               void* stream);

/* Size of the device scratch array behind vk_gemm_noalloc: the largest
 * workspace any version plans on a device of up to 256 CUs (version 9's 256
 * split-tail pieces of 256 KiB plus their counters; version 8's split-K
 * partials stay within 32 MiB, version 11's k-slices within 16 MiB), with
 * room to spare. */
#define VK_GEMM_SCRATCH_BYTES ((size_t)64 * 1024 * 1024 + (size_t)64 * 1024)

/* Same as vk_gemm, but allocates nothing (no hipMalloc or hipFree, no host
 * allocation): a version that needs a workspace uses the library's scratch
 * array of VK_GEMM_SCRATCH_BYTES in device memory, one copy per device, which
 * each device that runs the library holds until the process ends.  A plan
 * needing more returns VK_ERR_WORKSPACE.  The counters in it are cleared by a
 * small kernel in every call; every call on one device shares that device's
 * scratch, so calls that overlap on one device race (issue them on one
 * stream).  No counterpart in the reference: for callers that cannot
 * allocate -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc. */
int vk_gemm_noalloc(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n, size_t k,
                    const void* A, const void* B, void* C, void* stream);

/* Workspace bytes a call of this version and shape needs on the current
 * device (0: none).  Versions 8 to 14 depend on the device's
 * compute-unit count;
 * with no device to ask, an MI355X's 256 CUs are assumed.  No counterpart in
 * the reference, whose versions keep such buffers in function-local statics
 * (matmul_f16_v42_shfl2.cu:496-519). */
size_t vk_gemm_workspace_bytes(int version, vk_dtype in_dtype, size_t m, size_t n, size_t k);

/* Short name of a version ("f16_v2_dma256", ...), or NULL if unknown. */
const char* vk_gemm_name(int version, vk_dtype in_dtype);

/* Fill *caps; VK_ERR_VERSION if unknown. */
int vk_gemm_query(int version, vk_dtype in_dtype, vk_caps* caps);

/* Write up to max_count version ids for in_dtype into out; return how many
 * exist.  fp16 versions VK_F16_LEAVE_ONE_OUT_FIRST .. _LAST are version 7
 * with one ingredient of its k-loop or tile order turned off each (71: A
 * swizzle, 72: B swizzle, 73: direct-to-LDS loads replaced by VGPR staging,
 * 74: B ring cut to 2 slots, 75: no ping-pong, 76: no XCD-aware tile order,
 * 77: no accumulator chains of 2); they exist to be measured against
 * version 7 (bitwise equal results, same shapes accepted) and have no
 * counterpart in the reference. */
#define VK_F16_LEAVE_ONE_OUT_FIRST 71
#define VK_F16_LEAVE_ONE_OUT_LAST 77
int vk_gemm_list(vk_dtype in_dtype, int* out, int max_count);

/* Check a call without launching: the same validation vk_gemm performs. */
int vk_gemm_check(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n, size_t k,
                  const void* A, const void* B, const void* C);

/* Free library-managed workspaces on every device. */
int vk_gemm_release(void);

const char* vk_status_string(int status);
int vk_gemm_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* VK_GEMM_H */
