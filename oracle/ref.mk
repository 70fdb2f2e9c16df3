# Builds the reference's own CPU path into oracle/_ref/libriemann_ref.so
# (test infrastructure: the tests check the oracle and the HIP path against
# it; bench.py times it as the CPU baseline).
#
# The reference sources are compiled where they lie (nothing is copied): the
# coordinate manager (space.cpp), the stencil generator (stencil.cpp), the
# convolution and pooling layers (conv.cpp, pooling.cpp) and SparseTensor
# (sparse_tensor.cpp), with CPU_ONLY, against the LibTorch headers and
# libraries of the installed torch.
# The only source of this repository in the library is ref_driver.cpp, which
# calls the reference's public C++ API. Outputs go to oracle/_ref/ only.
#
#   make -f oracle/ref.mk            (from the repository root)
#   make -f oracle/ref.mk REF=/path/to/reference
REF ?= /root/reference
HERE := $(dir $(lastword $(MAKEFILE_LIST)))
OUT := $(HERE)_ref
TORCH := $(shell python3 -c "import os, torch; print(os.path.dirname(torch.__file__))")

CXX := g++
CXXFLAGS := -std=c++20 -O2 -fPIC -fopenmp -DCPU_ONLY -DRIEMANN_NO_PYBIND \
	-D_GLIBCXX_USE_CXX11_ABI=1 -w \
	-I$(REF) -I$(REF)/RiemannEngine -I$(REF)/RiemannEngine/vendor \
	-I$(TORCH)/include -I$(TORCH)/include/torch/csrc/api/include
LDFLAGS := -shared -fopenmp -L$(TORCH)/lib -ltorch -ltorch_cpu -lc10 \
	-Wl,-rpath,$(TORCH)/lib -Wl,--no-undefined

REF_SRCS := grid/space.cpp grid/stencil.cpp nn/conv.cpp nn/pooling.cpp tensor/sparse_tensor.cpp
REF_OBJS := $(addprefix $(OUT)/,$(subst /,_,$(REF_SRCS:.cpp=.o)))

all: $(OUT)/libriemann_ref.so

$(OUT)/grid_%.o: $(REF)/RiemannEngine/engine/grid/%.cpp
	@mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/nn_%.o: $(REF)/RiemannEngine/engine/nn/%.cpp
	@mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/tensor_%.o: $(REF)/RiemannEngine/engine/tensor/%.cpp
	@mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/ref_driver.o: $(HERE)ref_driver.cpp
	@mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/libriemann_ref.so: $(REF_OBJS) $(OUT)/ref_driver.o
	$(CXX) -o $@ $^ $(LDFLAGS)

clean:
	rm -rf $(OUT)

.PHONY: all clean
