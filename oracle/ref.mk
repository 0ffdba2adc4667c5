# Builds the reference C sources, where they lie under /root/reference, into
# oracle/_ref/libspref.so (plus this directory's ref_harness.c, which drives
# them).  Nothing is copied; outputs go to oracle/_ref/ only.  Used to pin the
# oracle; never part of the product.  gnu11 -O2 on baseline x86-64 (no FMA).
REF  ?= /root/reference
ORC  := $(abspath $(dir $(lastword $(MAKEFILE_LIST))))
OUT  := $(ORC)/_ref
CC   ?= gcc
SRC  := \
  core/forward_kernels/forward_kernels.c core/exact_islands/exact_islands.c \
  core/io_hash/sp_hash.c core/io_format/sp_model_load.c core/io_format/sp_model_arch.c \
  core/io_format/sp_error.c core/weight_dtype/weight_dtype.c core/gguf/gguf.c \
  core/ntt_crt/ntt_crt.c core/ntt_crt/ntt_batch.c core/poly_ring/poly_ring.c \
  core/poly_ring/poly_ring_bluestein.c core/poly_ring/resdot.c \
  core/vht2/spinor_block.c core/vht2/vht2.c core/vht2/mobius_reorder.c \
  core/frobenius/frobenius_lift.c core/kste/kste_encode.c core/kste/kste_dominance.c \
  core/arena/arena.c core/model/model.c core/forward_dispatch/forward_dispatch.c \
  core/arm/arm.c core/arm/arm_scan.c \
  core/forward/forward.c core/forward/decode.c core/forward/gemma3.c core/forward/gemma4.c \
  core/forward/qwen25.c core/forward/qwen36.c core/forward/generate.c \
  core/session/sp_session.c core/session/sp_model_bridge.c \
  core/session/qwen3_fixture.c core/session/gemma3_fixture.c
OBJ := $(patsubst %.c,$(OUT)/obj/%.o,$(SRC))
CFLAGS := -std=gnu11 -O2 -fPIC -w -I$(REF)/include -I$(REF)/core/session

$(OUT)/libspref.so: $(OBJ) $(ORC)/ref_harness.c
	$(CC) $(CFLAGS) -shared -Wl,-Bsymbolic -o $@ $(OBJ) $(ORC)/ref_harness.c -lm -lpthread

$(OUT)/obj/%.o: $(REF)/%.c
	@mkdir -p $(dir $@)
	$(CC) $(CFLAGS) -c $< -o $@
