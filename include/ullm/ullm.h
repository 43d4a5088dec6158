/* ullm/ullm.h -- umbrella header (reference include/ullm/ullm.h:1-6), extended
 * with the linear-layer entry points of this build. */
#ifndef ULLM_ULLM_H
#define ULLM_ULLM_H

#include "ullm/hip.h"
#include "ullm/linear.h"

#endif /* ULLM_ULLM_H */
