// Decode kernels instantiated for one KV dtype (see decode_impl.h).
#include "decode_impl.h"

template int dd_decode::dispatch_d<DD_F32, DD_F32>(const dd_decode::DecodeParams &, int, hipStream_t, int);
