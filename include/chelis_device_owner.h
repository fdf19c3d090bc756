/* Opaque device tensor owner: the C ABI of
 * crates/chelis-backend-hip/runtime/chelis_device_owner.h:16-24, same names,
 * argument meaning and trap behaviour (every invalid input traps `domain`
 * or `overflow` in metadata_plan; a HIP failure aborts). Implemented in
 * chelis_amd/csrc/device_owner.hip. Differences are internal only: clone
 * and strided host copies run as one device gather on the library stream
 * instead of one hipMemcpy per element. */
#ifndef CHELIS_DEVICE_OWNER_H
#define CHELIS_DEVICE_OWNER_H

#include "chelis_runtime.h"
#include "chelis_device_descriptor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct chelis_device_tensor_owner chelis_device_tensor_owner;

/* chelis_device_owner.h:16: takes the plan; zero-filled owned storage. */
chelis_device_tensor_owner *chelis_device_tensor_alloc(chelis_metadata_plan *plan);
/* chelis_device_owner.h:17: takes the plan; borrows device storage. */
chelis_device_tensor_owner *chelis_device_tensor_borrow(chelis_metadata_plan *plan, void *data, chelis_scalar byte_capacity);
/* chelis_device_owner.h:18: borrows a foreign packet (ownership must be 0). */
chelis_device_tensor_owner *chelis_device_tensor_import(const chelis_gpu_tensor *packet);
/* chelis_device_owner.h:19-20 */
const chelis_gpu_tensor *chelis_device_tensor_view(const chelis_device_tensor_owner *owner);
int32_t chelis_device_tensor_device(const chelis_device_tensor_owner *owner);
/* chelis_device_owner.h:21: an owned contiguous copy. */
chelis_device_tensor_owner *chelis_device_tensor_clone(const chelis_device_tensor_owner *source);
/* chelis_device_owner.h:22 */
void chelis_device_tensor_release(chelis_device_tensor_owner *owner);
/* chelis_device_owner.h:23-24 */
void chelis_device_tensor_copy_from_host(chelis_device_tensor_owner *destination, const chelis_tensor *source);
void chelis_device_tensor_copy_to_host(chelis_tensor_write *destination, const chelis_device_tensor_owner *source);

#ifdef __cplusplus
}
#endif
#endif
