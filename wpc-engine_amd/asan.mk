# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build of the
# library, for CPU tests of the parsers that read untrusted files
# (meta_json.cpp, json.cpp, safetensors.cpp) and of the transcoder and
# encoder: _build/asan/libwpcg_asan.so. Only the host C++ is instrumented (a host
# compiler, no .hip file on any of these lines); the gfx950 kernels are the normal
# build's objects, linked unchanged. The host compiler is ROCm's clang++
# (gcc 11 has no _Float16 in C++), with its shared sanitizer runtime; load
# the library with that runtime preloaded into an uninstrumented Python
# (tests/test_sanitize.py).
#   make -f asan.mk
ROCM    ?= /opt/rocm
CXX_ASAN := $(ROCM)/llvm/bin/clang++
SANFL   := -fsanitize=address,undefined -fno-sanitize-recover=all -fno-omit-frame-pointer -shared-libasan
FLAGS   := -O1 -g -std=c++17 -fPIC -ffp-contract=off -D__HIP_PLATFORM_AMD__ -I$(ROCM)/include $(SANFL)
HOSTSRC := $(wildcard csrc/*.cpp)
HIPOBJ  := $(patsubst csrc/%.hip,_build/%.hip.o,$(wildcard csrc/*.hip))
OBJS    := $(HOSTSRC:csrc/%.cpp=_build/asan/%.o)
LIB     := _build/asan/libwpcg_asan.so

all: $(LIB)

_build/asan/%.o: csrc/%.cpp csrc/wpcg_internal.hpp csrc/ref_expf.h ../include/wpcg.h
	@mkdir -p _build/asan
	$(CXX_ASAN) $(FLAGS) -c $< -o $@

$(HIPOBJ):
	$(MAKE) -f Makefile $@

$(LIB): $(OBJS) $(HIPOBJ)
	@mkdir -p lib
	$(CXX_ASAN) -shared $(SANFL) -o $@ $(OBJS) $(HIPOBJ) -L$(ROCM)/lib -Wl,-rpath,$(ROCM)/lib -lamdhip64 -lpthread

.PHONY: all
