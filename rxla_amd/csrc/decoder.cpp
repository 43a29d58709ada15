// Decoder plan (filled in later).
#include "internal.h"
using namespace rxw8;
extern "C" {
int rxw8_decoder_create(rxw8_runtime *, const rxw8_decoder_config *, rxw8_decoder **) {
  return fail(RXW8_UNIMPLEMENTED, "decoder not built yet");
}
int rxw8_decoder_destroy(rxw8_decoder *) { return fail(RXW8_UNIMPLEMENTED, "decoder not built yet"); }
int rxw8_decoder_num_parameters(rxw8_decoder *, int *) { return fail(RXW8_UNIMPLEMENTED, "decoder not built yet"); }
int rxw8_decoder_parameter_info(rxw8_decoder *, int, const char **, int *, int64_t *, int *) { return fail(RXW8_UNIMPLEMENTED, "decoder not built yet"); }
int rxw8_decoder_bind_parameter(rxw8_decoder *, const char *, rxw8_buffer *) { return fail(RXW8_UNIMPLEMENTED, "decoder not built yet"); }
int rxw8_decoder_reset(rxw8_decoder *) { return fail(RXW8_UNIMPLEMENTED, "decoder not built yet"); }
int rxw8_decoder_forward(rxw8_decoder *, rxw8_buffer *, int64_t, int64_t, rxw8_buffer *, rxw8_buffer *) { return fail(RXW8_UNIMPLEMENTED, "decoder not built yet"); }
int rxw8_decoder_generate(rxw8_decoder *, rxw8_buffer *, int64_t, int64_t, int64_t, rxw8_buffer *, int) { return fail(RXW8_UNIMPLEMENTED, "decoder not built yet"); }
int rxw8_decoder_lens(rxw8_decoder *, int32_t *, int64_t) { return fail(RXW8_UNIMPLEMENTED, "decoder not built yet"); }
}
