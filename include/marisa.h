// marisa.h -- umbrella header of the drop-in C++ surface.
#ifndef MARISA_H_
#define MARISA_H_

#include "marisa/base.h"
#include "marisa/keyset.h"
#include "marisa/tbs_input.h"
#include "marisa/trie.h"

#endif  // MARISA_H_
