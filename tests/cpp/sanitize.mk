# Host sanitizer build and fuzz of the backend's parsers (CPU only; nothing
# here runs on a GPU). From the repository root:
#
#   make -f tests/cpp/sanitize.mk check             build, then a short seeded fuzz of every mode
#   make -f tests/cpp/sanitize.mk check ITERS=20000  a longer one
#
# _san/host_fuzz: tests/cpp/host_fuzz.c with the library's host C sources and
# the driver's sources, built with AddressSanitizer and
# UndefinedBehaviorSanitizer (float-to-int overflow included), every report
# fatal. _san/lib/libtg_hip.so and _san/bin/tgc-hip: the library and driver
# with the same host objects instrumented (the HIP objects are the ordinary
# build's), for running the CPU test suite under the sanitizers:
#
#   make -f tests/cpp/sanitize.mk pytest
CC      ?= gcc
HIPCC   ?= /opt/rocm/bin/hipcc
ARCH    ?= gfx950
SEED    ?= 1
ITERS   ?= 3000
OUT      = _san
SRC      = technograd_amd/csrc
SAN      = -fsanitize=address,undefined,float-cast-overflow -fno-sanitize-recover=all -fno-omit-frame-pointer
CFLAGS_S = -std=gnu11 -O1 -g -fPIC -pthread -ffp-contract=off -Wall -Wno-unused-function -Iinclude -I$(SRC) $(SAN)
HOST_C   = tgir_read tgir_write tg_quant tg_gptq tg_front
HIP_OBJ  = tg_hip tg_decode tg_rpgen kern_layer kern_qgemm kern_rowprog kern_decode
export ASAN_OPTIONS  = detect_leaks=1:abort_on_error=1
export UBSAN_OPTIONS = print_stacktrace=1:halt_on_error=1

all: $(OUT)/host_fuzz $(OUT)/lib/libtg_hip.so $(OUT)/bin/tgc-hip

$(OUT)/obj/%.o: $(SRC)/%.c $(SRC)/tgm.h $(SRC)/tg_front.h $(SRC)/tg_gptq.h include/tg_hip.h
	@mkdir -p $(OUT)/obj
	$(CC) $(CFLAGS_S) -c -o $@ $<

$(OUT)/host_fuzz: tests/cpp/host_fuzz.c $(HOST_C:%=$(OUT)/obj/%.o) $(SRC)/tgc_hip_main.c $(SRC)/tgc_hip_serve.c
	$(CC) $(CFLAGS_S) -o $@ tests/cpp/host_fuzz.c $(HOST_C:%=$(OUT)/obj/%.o) -lm -lpthread

# the same harness under ThreadSanitizer, for the threaded parts (the server's
# batcher and connections, the batch driver's reader and writer)
$(OUT)/host_fuzz_tsan: tests/cpp/host_fuzz.c $(HOST_C:%=$(SRC)/%.c) $(SRC)/tgc_hip_main.c $(SRC)/tgc_hip_serve.c
	$(CC) -std=gnu11 -O1 -g -pthread -ffp-contract=off -Iinclude -I$(SRC) -fsanitize=thread -o $@ tests/cpp/host_fuzz.c \
	    $(HOST_C:%=$(SRC)/%.c) -lm -lpthread

# the ordinary build's HIP objects, linked with the instrumented host objects;
# the sanitizer runtimes come from the driver (or LD_PRELOAD under Python)
$(OUT)/lib/libtg_hip.so: $(HOST_C:%=$(OUT)/obj/%.o) $(HIP_OBJ:%=technograd_amd/build/%.o)
	@mkdir -p $(OUT)/lib
	$(HIPCC) --offload-arch=$(ARCH) -shared -pthread -o $@ $^ -lhiprtc

$(OUT)/bin/tgc-hip: $(SRC)/tgc_hip_main.c $(SRC)/tgc_hip_serve.c $(OUT)/lib/libtg_hip.so
	@mkdir -p $(OUT)/bin
	$(CC) $(CFLAGS_S) -o $@ $(SRC)/tgc_hip_main.c $(SRC)/tgc_hip_serve.c -L$(OUT)/lib -ltg_hip -Wl,-rpath,'$$ORIGIN/../lib' -lm -lpthread

check: $(OUT)/host_fuzz $(OUT)/host_fuzz_tsan
	$(OUT)/host_fuzz tgir $(SEED) $(ITERS) tests/golden/haltm_f32.tgir tests/golden/opsmix_f32.tgir tests/golden/latent_q4g.tgir \
	    tests/golden/ssm_small_q8.tgir tests/golden/qmlp_q4.tgir tests/golden/latent_f32.tgir
	$(OUT)/host_fuzz front $(SEED) $(ITERS) tests/golden/front/*.tg tests/golden/models/*.tg
	$(OUT)/host_fuzz gptq $(SEED) $$(( $(ITERS) / 20 + 1 )) tests/golden/qmlp_f32.tgir tests/golden/latent_f32.tgir tests/golden/haltm_f32.tgir
	$(OUT)/host_fuzz rows $(SEED) $$(( $(ITERS) * 10 ))
	$(OUT)/host_fuzz http $(SEED) $(ITERS) tests/golden/latent_f32.tgir
	$(OUT)/host_fuzz cli $(SEED) $$(( $(ITERS) / 10 + 1 )) tests/golden/latent_f32.tgir
	$(OUT)/host_fuzz cli $(SEED) $$(( $(ITERS) / 10 + 1 )) tests/golden/qmlp_q4.tgir
	TSAN_OPTIONS=halt_on_error=1 $(OUT)/host_fuzz_tsan http $(SEED) $$(( $(ITERS) / 4 + 1 )) tests/golden/latent_f32.tgir
	TSAN_OPTIONS=halt_on_error=1 $(OUT)/host_fuzz_tsan cli $(SEED) $$(( $(ITERS) / 20 + 1 )) tests/golden/latent_f32.tgir

# the CPU tests that drive the host code, against the instrumented library and driver
pytest: $(OUT)/lib/libtg_hip.so $(OUT)/bin/tgc-hip
	ASAN_OPTIONS=detect_leaks=0:abort_on_error=1 TG_HIP_LIB=$(abspath $(OUT)/lib/libtg_hip.so) TGC_HIP=$(abspath $(OUT)/bin/tgc-hip) \
	LD_PRELOAD="$$($(CC) -print-file-name=libasan.so) $$($(CC) -print-file-name=libubsan.so)" \
	    python -m pytest -x -q -p no:cacheprovider -m "not gpu" tests/test_host.py tests/test_front.py tests/test_quantize.py tests/test_cli.py tests/test_rpgen.py

clean:
	rm -rf $(OUT)

.PHONY: all check pytest clean
