/*
 * sfa.h -- tensor descriptors shared by the cf_hip C ABI and its callers.
 *
 * The descriptor layout is the MLIR memref descriptor that the reference's
 * Stable Function ABI uses (reference include/sfa.h:54-99):
 *
 *     { void* allocated; void* aligned; int64 offset;
 *       int64 sizes[R]; int64 strides[R]; }          (24 + 16 R bytes)
 *
 * Strides and the offset are counted in ELEMENTS, not bytes (reference
 * compiler/dylib_ffi.py:46-55).  The layout must stay byte-identical so a
 * caller that already builds SFA descriptors (Python ctypes, the Rust
 * SfaMemRef, compiled MLIR code) can hand them to this library unchanged.
 *
 * One value is added to SFADevice: SFA_ROCM = 3 marks device memory of the
 * current HIP device.  SFA_CPU = 1 and SFA_CUDA = 2 keep their numbers.
 */
#ifndef CF_SFA_H
#define CF_SFA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    SFA_CPU = 1,
    SFA_CUDA = 2,
    SFA_ROCM = 3,
} SFADevice;

typedef struct {
    void* allocated;
    void* aligned;
    int64_t offset;
    int64_t sizes[1];
    int64_t strides[1];
} SFATensorRaw1;

typedef struct {
    void* allocated;
    void* aligned;
    int64_t offset;
    int64_t sizes[2];
    int64_t strides[2];
} SFATensorRaw2;

typedef struct {
    void* allocated;
    void* aligned;
    int64_t offset;
    int64_t sizes[3];
    int64_t strides[3];
} SFATensorRaw3;

typedef struct {
    void* allocated;
    void* aligned;
    int64_t offset;
    int64_t sizes[4];
    int64_t strides[4];
} SFATensorRaw4;

typedef struct {
    SFADevice device;
    int32_t rank;
    int32_t elem_size; /* bytes per element */
    union {
        SFATensorRaw1 r1;
        SFATensorRaw2 r2;
        SFATensorRaw3 r3;
        SFATensorRaw4 r4;
    };
} SFATensor;

#ifdef __cplusplus
}
#endif

#endif /* CF_SFA_H */
