/* ullm/ullm.h -- umbrella header (reference include/ullm/ullm.h:1-6), extended
 * with the linear-layer and weight-file entry points of this build. */
#ifndef ULLM_ULLM_H
#define ULLM_ULLM_H

#include "ullm/hip.h"
#include "ullm/linear.h"
#include "ullm/weights_io.h"

#endif /* ULLM_ULLM_H */
