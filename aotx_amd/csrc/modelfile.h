/* The GGUF reader and descriptor builder (modelfile.cpp, desc_file.cpp). */
#ifndef AOTX_MODELFILE_INTERNAL_H
#define AOTX_MODELFILE_INTERNAL_H

#include "../../include/aotx_modelfile.h"

#endif
