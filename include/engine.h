/* Ijah-compatible C API on MI355X (HIP). Plain C for ctypes / any FFI.
 *
 * Every declaration here keeps the name, signature, struct layout and error convention of the reference's
 * include/engine.h (publicExcess/ijah), so tools/engine.py binds this library unchanged; each line cites the
 * reference declaration it replaces. Where the semantics differ on a discrete GPU it is said beside the function.
 *
 * Conventions (reference include/engine.h:3-12)
 * - int functions: 0 = ok, -1 = error, message in ne_last_error() (per thread). Pointer functions: NULL = error.
 * - Buffers live in HBM. ne_buf_contents() returns a host mirror refreshed from the device at that call (the
 *   reference's unified memory has no copy). Bytes the caller changes in the mirror reach the GPU before the next
 *   library call that uses the buffer (a kernel or hot-path run, an upload, a download, ne_buf_contents itself),
 *   and only the changed bytes, so the reference's write-then-run pattern works; ne_buf_flush() (ijah_exl3.h)
 *   writes the whole mirror at once. A caller that reads results must call ne_buf_contents() again after the run
 *   (the GPU's writes do not reach an existing mirror), and must not change bytes the GPU is still writing.
 *   Exception: a call made while the library's stream is being captured into a graph pushes nothing (a copy would
 *   be recorded into the graph): call ne_buf_flush() before the capture.
 * - Pack tensors are uploaded to HBM on first use; their ne_buf handles belong to the pack (do not ne_free them).
 */
#ifndef NATIVE_ENGINE_H
#define NATIVE_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NE_API __attribute__((visibility("default")))
#define NE_ABI_VERSION 1

/* dtype values: reference include/engine.h:28-31 (same numbers) */
typedef enum {
  NE_F32 = 0, NE_F16 = 1, NE_BF16 = 2, NE_U8 = 3, NE_U16 = 4, NE_U32 = 5, NE_I32 = 6,
  NE_I64 = 7, NE_I8 = 8, NE_I16 = 9, NE_U64 = 10, NE_F64 = 11, NE_BOOL = 12
} ne_dtype;
#define NE_MAX_DIMS 8

NE_API int ne_abi_version(void);             /* reference include/engine.h:34 */
NE_API const char *ne_last_error(void);      /* reference include/engine.h:35 */
NE_API const char *ne_dtype_name(int dtype); /* reference include/engine.h:36 */
NE_API int ne_dtype_size(int dtype);         /* reference include/engine.h:37 */

/* reference include/engine.h:40-49 (same layout). On MI355X: has_nax = 1 (MFMA matrix cores), has_metal4 = 0,
 * backend = "hip". */
typedef struct {
  char name[64];
  int has_nax;
  int has_metal4;
  uint64_t max_buffer_length;
  uint64_t recommended_working_set;
  uint64_t max_threadgroup_memory;
  char backend[16];
} ne_device_info;
NE_API int ne_device_query(ne_device_info *out); /* reference include/engine.h:49 */

typedef struct ne_buf ne_buf;
NE_API ne_buf *ne_alloc(uint64_t nbytes);                   /* reference include/engine.h:53: HBM, zero-filled */
NE_API void ne_free(ne_buf *b);                             /* reference include/engine.h:54 */
NE_API uint64_t ne_buf_size(const ne_buf *b);               /* reference include/engine.h:55 */
NE_API void *ne_buf_contents(const ne_buf *b);              /* reference include/engine.h:56: host mirror, see top */
NE_API uint64_t ne_buf_gpu_address(const ne_buf *b);        /* reference include/engine.h:57: device address */
NE_API int ne_upload(ne_buf *b, uint64_t offset, const void *src, uint64_t nbytes);  /* reference :58 */
NE_API int ne_download(const ne_buf *b, uint64_t offset, void *dst, uint64_t nbytes); /* reference :59 */

/* packs: a directory of safetensors shards + config.json (reference include/engine.h:62-83, same layout) */
typedef struct ne_pack ne_pack;
typedef struct {
  int dtype;
  int ndim;
  int64_t shape[NE_MAX_DIMS];
  uint64_t nbytes;
  const char *file;
  uint64_t file_offset;
  const void *host;
  ne_buf *buf;
  uint64_t buf_offset;
} ne_tensor_desc;

NE_API ne_pack *ne_pack_open(const char *dir);                        /* reference include/engine.h:75 */
NE_API void ne_pack_close(ne_pack *p);                                /* reference include/engine.h:76 */
NE_API const char *ne_pack_config_json(const ne_pack *p);             /* reference include/engine.h:77 */
NE_API int64_t ne_pack_num_tensors(const ne_pack *p);                 /* reference include/engine.h:78 */
NE_API const char *ne_pack_tensor_name(const ne_pack *p, int64_t i);  /* reference include/engine.h:79 */
NE_API int ne_tensor_info(const ne_pack *p, const char *name, ne_tensor_desc *out); /* reference :80 */
NE_API ne_buf *ne_pack_view_rows(const ne_pack *p, const char *name, int64_t row0, int64_t nrows,
                                 uint64_t *offset);                   /* reference include/engine.h:83 */

/* kernels by name (reference include/engine.h:85-98). Function constants select a registered instantiation
 * (index 10 = K, index 16 = R); grid counts workgroups, tg = threads per workgroup (multiple of 64), tg_mem = dynamic
 * LDS bytes. backend must be NULL, "" or "hip". */
typedef struct { uint32_t index; uint32_t type; uint32_t bits; } ne_fconst;
typedef struct { ne_buf *buf; uint64_t offset; const void *bytes; uint32_t nbytes; } ne_arg;

NE_API int ne_kernel_exists(const char *fn);                          /* reference include/engine.h:92 */
NE_API int ne_run_kernel(const char *fn, const ne_fconst *fc, int nfc, const ne_arg *args, int nargs,
                         const uint32_t grid[3], const uint32_t tg[3], uint32_t tg_mem, int reps,
                         const char *backend, double *gpu_ms);        /* reference include/engine.h:96-98 */

#ifdef __cplusplus
}
#endif
#endif /* NATIVE_ENGINE_H */
