// Decode kernels instantiated for one KV dtype (see decode_impl.h).
#include "decode_impl.h"

template int dd_decode::dispatch_d<DD_BF16, DD_BF16>(const dd_decode::DecodeParams &, int, hipStream_t, int);
