// Per-(device, stream) decode state kept in device memory by the library.
#pragma once

#include <stdint.h>

namespace qmk {

struct DecodeState {
  uint32_t epoch;  // exchange-tag base; advanced by every completed launch
  uint32_t err;    // error bits (0 = healthy); a non-zero value makes launches no-ops
  int32_t eos;     // persistent mode: stop token (-1: none)
  uint32_t done;   // persistent mode: `eos` was emitted; later launches only pad the log with it
  int32_t pos;     // persistent mode: position, input token and step of the next launch
  int32_t tok;
  int32_t step;
  int32_t ran;     // persistent mode: 1 if the last launch decoded a token, 0 if it only padded the log
  uint32_t reserved[56];  // header is 256 bytes; exchange words follow
};
static_assert(sizeof(DecodeState) == 256, "state header size");

}  // namespace qmk
