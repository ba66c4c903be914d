/* Instantiates the reference's single-header C decoder (ref/c/hct_decoder.h)
 * as a shared library, as that header's usage notes prescribe.  Built by
 * oracle/Makefile into oracle/_ref/ only; test infrastructure. */
#define HCT_IMPLEMENTATION
#include "hct_decoder.h"
