/* Oracle translation unit — TEST INFRASTRUCTURE ONLY (see oracle_body.h).
 * Instantiates the restatement at f32 (orc32_*) and f64 (orc64_*). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define REAL float
#define PFX orc32_
#include "oracle_body.h"
#undef REAL
#undef PFX

#define REAL double
#define PFX orc64_
#include "oracle_body.h"
#undef REAL
#undef PFX
