'''motif: MI355X-native (gfx950) implementation of Motif Chord's sequence-mixing path.

Hand-written HIP kernels (libmotif_hip.so, C ABI in include/motif_hip.h) behind
the reference's `motif.ops` functions and the GatedDeltaAttention /
ChordAttention layer interfaces.
'''
