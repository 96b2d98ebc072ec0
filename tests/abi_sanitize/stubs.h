// What the launch stand-ins of stubs.cpp recorded.
#pragma once
#include "internal.h"

namespace stub {
extern kls::Args last_args;
extern kls::HeadArgs last_head;
extern int launches;
extern int fills;
extern unsigned char scratch[];
extern size_t scratch_bytes;
}  // namespace stub
