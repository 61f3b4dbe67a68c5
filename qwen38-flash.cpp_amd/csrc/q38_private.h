/* q38_private.h — hooks between the host-side checkpoint loader and the C ABI library;
 * not part of the public interface. */
#ifndef Q38_PRIVATE_H
#define Q38_PRIVATE_H

#include "q38.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Sets the thread's q38_last_error() message. */
void q38_private_set_error(const char* msg);
/* The layer takes ownership of a hipMalloc'ed block holding its tensors (freed with it). */
void q38_private_layer_adopt(q38_moe_layer* layer, void* device_block);

#ifdef __cplusplus
}
#endif

#endif
