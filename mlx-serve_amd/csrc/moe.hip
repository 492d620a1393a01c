#include "mi_internal.h"
