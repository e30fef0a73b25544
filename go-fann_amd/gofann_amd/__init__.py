"""gofann_amd -- host side of the MI355X GPU stage of GO-FANN's filtered
graph search.  Kernels live in libgofann_hip.so (C ABI: include/gofann_hip.h);
this package binds it (_lib), builds synthetic indexes (synth, index), plans
routes (plan) and drives searches (search)."""
