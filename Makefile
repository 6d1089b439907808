# EdgeCore MI355X build.  Everything lands in-tree so it travels with the
# repository snapshot:
#   edgecore_amd/lib/libedgecore_hip.so   the C-ABI library (HIP, gfx950)
#   edgecore_amd/bin/edgecore-runtime     the command-line driver
#   edgecore_amd/bin/ecm_synth            seeded synthetic .ecm / prompt generator
#   oracle/liboracle.so                   CPU oracle (test infrastructure)
#   oracle/_ref/*                         reference CPU runtime built from its sources,
#                                         only where the reference tree exists
ROCM    ?= /opt/rocm
HIPCC   ?= $(ROCM)/bin/hipcc
CC      ?= gcc
ARCH    ?= gfx950
REF     ?= /root/reference

PKG     := edgecore_amd
SRC     := $(PKG)/csrc
OBJ     := build/obj
LIB     := $(PKG)/lib/libedgecore_hip.so
RUNTIME := $(PKG)/bin/edgecore-runtime
SYNTH   := $(PKG)/bin/ecm_synth

# -ffp-contract=off keeps every a*b+c a rounded multiply and a rounded add, as
# in the reference's -std=c11 build; packed fp32 instructions are disabled.
HIPFLAGS := --offload-arch=$(ARCH) -O3 -std=c++17 -fPIC -ffp-contract=off \
            -Xclang -target-feature -Xclang -packed-fp32-ops -Iinclude -I$(SRC) -Wall
CFLAGS   := -O2 -std=c11 -Wall -Wextra -fPIC -Iinclude -ffp-contract=off

HIPSRC := $(SRC)/kernels.hip $(SRC)/decode_step.hip $(SRC)/decode_step_gpt2.hip $(SRC)/decode_tail.hip $(SRC)/gemm_mfma.hip $(SRC)/attn_prefill.hip $(SRC)/topk.hip $(SRC)/gemv_i8.hip $(SRC)/gemv_f16.hip $(SRC)/gemv_bf16.hip $(SRC)/runtime.hip
HIPOBJ := $(HIPSRC:$(SRC)/%.hip=$(OBJ)/%.o)

all: $(LIB) $(RUNTIME) $(SYNTH) oracle

$(OBJ) $(PKG)/lib $(PKG)/bin:
	mkdir -p $@

$(OBJ)/%.o: $(SRC)/%.hip $(SRC)/ec_device.h $(SRC)/ec_kernels.h $(SRC)/attn_decode.h $(SRC)/gemv_impl.h $(SRC)/ec_expf.h $(SRC)/ec_quant.h $(SRC)/step_common.h include/edgecore.h | $(OBJ)
	$(HIPCC) $(HIPFLAGS) -c $< -o $@

$(OBJ)/ecm.o: $(SRC)/ecm.c include/edgecore.h | $(OBJ)
	$(CC) $(CFLAGS) -c $< -o $@

$(OBJ)/sample.o: $(SRC)/sample.c include/edgecore.h | $(OBJ)
	$(CC) $(CFLAGS) -c $< -o $@

$(OBJ)/tokenizer.o: $(SRC)/tokenizer.c include/edgecore.h | $(OBJ)
	$(CC) $(CFLAGS) -c $< -o $@

$(LIB): $(HIPOBJ) $(OBJ)/ecm.o $(OBJ)/sample.o $(OBJ)/tokenizer.o | $(PKG)/lib
	$(HIPCC) --offload-arch=$(ARCH) -shared -fPIC $^ -o $@

$(RUNTIME): $(SRC)/runtime_main.c include/edgecore.h $(LIB) | $(PKG)/bin
	$(CC) $(CFLAGS) $< -o $@ -L$(PKG)/lib -ledgecore_hip -Wl,-rpath,'$$ORIGIN/../lib' -lm

$(SYNTH): $(SRC)/ecm_synth.c $(SRC)/ecm.c include/edgecore.h | $(PKG)/bin
	$(CC) -O2 -std=c11 -Wall -Wextra -fopenmp -Iinclude $(SRC)/ecm_synth.c $(SRC)/ecm.c -o $@ -lm

oracle:
	$(MAKE) -C oracle
	@if [ -d "$(REF)/src" ]; then $(MAKE) -C oracle ref REF=$(REF); fi

clean:
	rm -rf build $(PKG)/lib $(PKG)/bin
	$(MAKE) -C oracle clean

.PHONY: all oracle clean
