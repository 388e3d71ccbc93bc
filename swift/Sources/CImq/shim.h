/* The C ABI of libimq.so for Swift: the five public headers of include/. */
#include "../../../include/imq.h"
#include "../../../include/imq_weights.h"
#include "../../../include/imq_step.h"
#include "../../../include/imq_cond.h"
#include "../../../include/imq_te.h"
