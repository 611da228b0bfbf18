"""C-ABI checks that need no GPU: the library loads, exports every entry
point include/catfuse_amd.h declares, and rejects malformed arguments on
the host (before any launch) with hipErrorInvalidValue."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "catfuse_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(cf_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("cf_lif_multistep", "cf_conv_mfma", "cf_prescan_tiles", "cf_pack_input",
              "cf_conv_direct", "cf_avgpool2x2_lif", "cf_route_from_nnz"):
        assert s in syms


def test_count_block_size_matches_header():
    from catfuse_amd import runtime
    m = re.search(r"#define CF_COUNT_BLOCK_WORDS (\d+)", open(HEADER).read())
    assert m and int(m.group(1)) == runtime.COUNT_BLOCK_WORDS
    src = open(os.path.join(ROOT, "catfuse_amd", "csrc", "cf_common.h")).read()
    groups = int(re.search(r"CF_COUNT_GROUPS = (\d+);", src).group(1))
    assert 16 * (groups + 1) == runtime.COUNT_BLOCK_WORDS


def test_library_exports_every_declared_symbol():
    from catfuse_amd import _hip
    path = _hip.library_path()
    assert os.path.exists(path), "build the library first (python -m catfuse_amd.build)"
    lib = ctypes.CDLL(path)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"not exported: {missing}"
    # and the Python binding covers them all
    assert set(declared_symbols()) <= set(_hip._SIGNATURES)


def test_version():
    from catfuse_amd import _hip
    assert _hip.lib().cf_version() >= 100


INVALID = 1  # hipErrorInvalidValue


def test_host_side_argument_validation():
    from catfuse_amd import _hip
    L = _hip.lib()
    # null input / bad mode
    assert L.cf_lif_multistep(None, None, None, None, 0, None, None, 0, None, 4, 16, 1, 1,
                              2.0, 1.0, 0.0, 1, 1, None) == INVALID
    assert L.cf_lif_multistep(1, None, None, None, 9, None, 1, 0, None, 4, 16, 1, 1,
                              2.0, 1.0, 0.0, 1, 1, None) == INVALID
    # add modes need z2, affine modes need scale/shift
    assert L.cf_lif_multistep(1, None, None, None, 3, None, 1, 0, None, 4, 16, 1, 1,
                              2.0, 1.0, 0.0, 1, 1, None) == INVALID
    assert L.cf_lif_multistep(1, None, None, None, 1, None, 1, 0, None, 4, 16, 1, 1,
                              2.0, 1.0, 0.0, 1, 1, None) == INVALID
    # conv: Cp not a multiple of 32
    assert L.cf_conv_mfma(1, 1, 1, 1, None, None, 1, None, 0, None, None, 0, 0, None, None, None, None,
                          None, None, None, 0, None, 0, 0.7,
                          4, 2, 48, 64, 64, 8, 8, 8, 8, 3, 3, 1, 1, 2, 0, 0, 0,
                          0, 2.0, 1.0, 0.0, 1, 1, None) == INVALID
    # conv: inconsistent output size
    assert L.cf_conv_mfma(1, 1, 1, 1, None, None, 1, None, 0, None, None, 0, 0, None, None, None, None,
                          None, None, None, 0, None, 0, 0.7,
                          4, 2, 64, 64, 64, 8, 8, 7, 8, 3, 3, 1, 1, 2, 0, 0, 0,
                          0, 2.0, 1.0, 0.0, 1, 1, None) == INVALID
    # conv: rect tile must hold 64 or 128 pixels
    assert L.cf_conv_mfma(1, 1, 1, 1, None, None, 1, None, 0, None, None, 0, 0, None, None, None, None,
                          None, None, None, 0, None, 0, 0.7,
                          4, 2, 64, 64, 64, 8, 8, 8, 8, 3, 3, 1, 1, 2, 4, 4, 16,
                          0, 2.0, 1.0, 0.0, 1, 1, None) == INVALID
    # conv: a tile order needs tile masks
    assert L.cf_conv_mfma(1, 1, 1, 1, None, None, 1, None, 0, None, None, 0, 0, None, 1, None, None,
                          None, None, None, 0, None,
                          0, 0.7, 4, 2, 64, 64, 64, 8, 8, 8, 8, 3, 3, 1, 1, 2, 8, 8, 16,
                          0, 2.0, 1.0, 0.0, 1, 1, None) == INVALID
    # conv: bias knowledge needs an output descriptor; unknown bits
    for x_desc, out_desc, info in ((None, None, 1), (None, None, 2), (None, 1, 4)):
        assert L.cf_conv_mfma(1, 1, 1, 1, None, None, 1, 1, 64, None, None, 0, 0, None, None, None,
                              None, x_desc, None, out_desc, info, None,
                              0, 0.7, 4, 2, 64, 64, 64, 8, 8, 8, 8, 3, 3, 1, 1, 2, 0, 0, 0,
                              0, 2.0, 1.0, 0.0, 1, 1, None) == INVALID
    # pooled epilogue (2): stride-1 3x3 convs on 8x8 tiles writing the fp16
    # copy only, whole 32-channel groups, no identity, no bias knowledge
    def pooled(out=None, identity=None, out_desc=None, info=0, Cout=64, cp_out=64, H=8, Ho=8,
               k=3, stride=1, pad=1, tiles=(0, 0, 0), ag=None, T=4, v_out=1, epi=2):
        return L.cf_conv_mfma(1, 1, 1, 1, None, v_out, out, 1, cp_out, identity, None, 64,
                              1, ag, None, None, None, None, None, out_desc, info, None, 0, 0.7,
                              T, 2, 64, Cout, 64, H, H, Ho, Ho, k, k, stride, pad, 2, *tiles,
                              epi, 2.0, 1.0, 0.0, 1, 1, None)
    assert pooled(out=1) == INVALID                          # fp32 output
    assert pooled(identity=1) == INVALID                     # identity
    assert pooled(Cout=48, cp_out=48) == INVALID             # partial 32-channel group
    assert pooled(Cout=32, cp_out=34) == INVALID             # copy pitch not a multiple of 4
    assert pooled(H=16, stride=2) == INVALID                 # stride 2
    assert pooled(k=1, pad=0) == INVALID                     # 1x1 kernel
    assert pooled(tiles=(8, 16, 16), ag=1) == INVALID        # 8x16 tiles
    assert pooled(H=1, Ho=1) == INVALID                      # no whole 2x2 window
    assert pooled(T=9, v_out=None) == INVALID                # state across time blocks
    assert pooled(epi=3) == INVALID                          # unknown epilogue
    assert L.cf_bias_response(1, 1, 0, 4, 0, 2.0, 1.0, 0.0, 1, 1, 1, 1, None) == INVALID
    assert L.cf_bias_response(1, None, 8, 4, 0, 2.0, 1.0, 0.0, 1, 1, 1, 1, None) == INVALID
    assert L.cf_bias_response(1, 1, 8, 4, 2, 2.0, 1.0, 0.0, 1, 1, 1, 1, None) == INVALID
    assert L.cf_conv_mfma(1, 1, 1, 1, None, None, 1, 1, 64, None, None, 0, 0, None, None, None, None,
                          None, None, None, 1, None,
                          0, 0.7, 4, 2, 64, 64, 64, 8, 8, 8, 8, 3, 3, 1, 1, 2, 0, 0, 0,
                          0, 2.0, 1.0, 0.0, 1, 1, None) == INVALID
    # descriptor resolution / state expansion: misaligned or partial units
    assert L.cf_resolve_copy(1, 24, 16, None) == INVALID
    assert L.cf_resolve_copy(8, 32, 16, None) == INVALID
    assert L.cf_resolve_copy(16, 32, None, None) == INVALID
    assert L.cf_expand_state(16, 16, None, 2, 4, 4, None) == INVALID
    assert L.cf_expand_state(16, 16, 16, 2, 0, 4, None) == INVALID
    # compaction: no tiles / no mask
    assert L.cf_compact_tiles(1, 4, 0, 8, 0.0, -1.0, 0.0, 1, None) == INVALID
    assert L.cf_compact_tiles(None, 4, 8, 8, 0.0, -1.0, 0.0, 1, None) == INVALID
    assert L.cf_compact_tiles(1, 4, 8, 33, 0.0, -1.0, 0.0, 1, None) == INVALID   # > 32 groups
    assert L.cf_compact_tiles(1, 4, 8, 8, float("nan"), -1.0, 0.0, 1, None) == INVALID
    # paired conv: the 1x1 conv's output size differs from the 3x3 conv's
    def pair(Ho=8, Cout_a=64, pad_b=0, out_a=1):
        return L.cf_conv_halo_pair(1, None, None, 0, 4, 2, 64, 16, 16, Ho, Ho,
                                   1, 1, 1, None, 1, out_a, 64, None, None, 0, Cout_a, 64, 1,
                                   1, 1, 1, None, 1, 1, 64, None, None, 0, 64, 64, pad_b,
                                   2.0, 1.0, 0.0, 1, 1, None)
    assert pair(pad_b=1) == INVALID                 # 1x1/s2 with padding 1: 9x9 output
    assert pair(Ho=7) == INVALID                    # inconsistent output size
    assert pair(Cout_a=48) == INVALID               # outputs in whole 32-channel groups
    assert pair(out_a=None) == INVALID              # NHWC outputs required
    # prescan: more than 32 groups
    assert L.cf_prescan_tiles(1, 1, 8, 8, 8, 8, 3, 1, 1, 8, 8, 33, 1, 1, None) == INVALID
    # pack: groups must fit 32 bits
    assert L.cf_pack_input(1, 1, 1024, 4, 4, 1024, None, 1, 16, 1e-6, None, None,
                           None) == INVALID


def test_stale_library_refused(monkeypatch):
    """A library whose recorded source digest differs from the tree's sources
    is refused before any entry point is bound."""
    from catfuse_amd import _hip, build
    monkeypatch.setattr(build, "source_digest", lambda: "0" * 64)
    monkeypatch.setattr(_hip, "_lib", None)
    with pytest.raises(RuntimeError, match="not built from the current sources"):
        _hip.lib()


def test_token_and_pool_entry_points_validate_arguments():
    """The Spikformer entry points reject shapes their kernels do not cover
    on the host, before any launch (pointers are placeholders: nothing is
    dereferenced)."""
    from catfuse_amd import _hip
    L = _hip.lib()
    lif = (2.0, 1.0, 0.0, 1, 1)

    def direct_pool(Cin=3, Cout=48, cp_out=64, pad=1, H=32, W=32):
        return L.cf_conv_direct_lif_maxpool(1, 1, 1, 1, None, None, 1, cp_out, None, 4, 2, Cin,
                                            Cout, H, W, pad, 0, *lif, None)
    assert direct_pool(Cin=5) == INVALID            # more than 4 input channels
    assert direct_pool(Cout=24, cp_out=32) == INVALID   # Cout not a multiple of 16
    assert direct_pool(cp_out=52) == INVALID        # copy pitch not a multiple of 8
    assert direct_pool(cp_out=32) == INVALID        # copy narrower than Cout
    assert direct_pool(pad=3) == INVALID            # padding beyond 2
    assert direct_pool(H=1, pad=0) == INVALID       # empty conv output

    def stem(Cin=3, KH=7, KW=7, stride=2, pad=3, T=4, pool=(3, 2, 1), cp_out=64):
        return L.cf_conv_stem_lif_maxpool(1, 1, 1, 1, None, None, None, 1, cp_out, None, None,
                                          T, 2, Cin, 64, 64, 64, 64, KH, KW, stride, pad,
                                          *pool, 2.0, 1.0, 0.0, 1, 1, None)
    assert stem(stride=3) == INVALID                # conv stride 1 or 2 only
    assert stem(T=33) == INVALID                    # spike trains up to 32 steps
    assert stem(Cin=5) == INVALID                   # at most 4 input channels
    assert stem(KH=8) == INVALID                    # filter rows up to 7
    assert stem(pool=(2, 2, 0)) == INVALID          # MaxPool2d(3, 2, 1) only
    assert stem(cp_out=60) == INVALID               # copy pitch a multiple of 8

    # head linear over a token copy: pitch below K, no outputs, too many outputs
    assert L.cf_linear_tokens(1, None, 1, None, 1, 4, 64, 32, 10, None) == INVALID
    assert L.cf_linear_tokens(1, None, 1, None, 1, 4, 64, 64, 0, None) == INVALID
    assert L.cf_linear_tokens(1, None, 1, None, 1, 4, 64, 64, 5000, None) == INVALID
    assert L.cf_linear_tokens(None, None, 1, None, 1, 4, 64, 64, 10, None) == INVALID

    def direct_avg(Cin=3, Cout=64, cp_out=64, pad=1, H=32, W=32):
        return L.cf_conv_direct_avgpool_lif(1, 1, 1, 1, None, None, 1, cp_out, None, 4, 2, Cin,
                                            Cout, H, W, pad, 0, 2.0, 1.0, 0.0, 1, 1, None)
    assert direct_avg(Cin=5) == INVALID             # more than 4 input channels
    assert direct_avg(Cout=24, cp_out=32) == INVALID    # Cout not a multiple of 16
    assert direct_avg(cp_out=68) == INVALID         # copy pitch not a multiple of 8
    assert direct_avg(cp_out=32) == INVALID         # copy narrower than Cout
    assert direct_avg(pad=3) == INVALID             # padding beyond 2
    assert direct_avg(H=3, pad=0) == INVALID        # 1-row conv output: no 2x2 window

    def attention(N=196, heads=2, head_dim=32, pitch=192, qoff=0, cp_out=64):
        return L.cf_spike_attention_lif(1, 1, 1, qoff, 64, 128, pitch, 1, cp_out, None, None,
                                        None, None, None, 0, 4, 2, N, heads, head_dim, 0.125,
                                        *lif, None)
    assert attention(head_dim=64) == INVALID        # one 32-wide MFMA tile per head
    assert attention(N=300) == INVALID              # more tokens than the kernel stages
    assert attention(qoff=160) == INVALID           # Q heads beyond the pitch
    assert attention(cp_out=32) == INVALID          # output narrower than heads * 32
    assert attention(pitch=196) == INVALID          # pitch not a multiple of 8
    assert L.cf_spike_attention_lif(1, 1, 1, 0, 64, 128, 192, 1, 64, None, None, None, None,
                                    None, 1, 4, 2, 196, 2, 32, 0.125, *lif,
                                    None) == INVALID    # zero-drive knowledge without a descriptor

    def pool(cp=64, k=3, s=2, p=1):
        return L.cf_maxpool_nhwc(1, None, 1, None, 8, 16, 16, cp, k, s, p, None, None)
    assert pool(cp=12) == INVALID                   # 16-byte channel chunks
    assert pool(k=2, p=2) == INVALID                # padding beyond half the window
    assert pool(s=0) == INVALID


def _header_struct_fields(name):
    text = open(HEADER).read()
    m = re.search(r"typedef struct " + name + r" \{(.*?)\} " + name + ";", text, re.S)
    assert m, name
    return [re.findall(r"(\w+);", line)[0] for line in m.group(1).strip().splitlines()
            if line.strip()]


@pytest.mark.parametrize("cname, pyname", [("CfConvMfmaArgs", "ConvMfmaArgs"),
                                           ("CfConvHaloPairArgs", "ConvHaloPairArgs")])
def test_argument_blocks_mirror_the_header(cname, pyname):
    """The ctypes mirrors of the argument blocks have the header's fields in
    the header's order, every one 8 bytes, and the library's sizeof."""
    from catfuse_amd import _hip
    st = getattr(_hip, pyname)
    assert [f for f, _ in st._fields_] == _header_struct_fields(cname)
    assert all(ctypes.sizeof(t) == 8 for _, t in st._fields_)
    sizes = (ctypes.c_int64 * 2)()
    assert _hip.lib().cf_conv_args_sizes(ctypes.addressof(sizes)) == 0
    assert ctypes.sizeof(st) == sizes[0 if cname == "CfConvMfmaArgs" else 1]
    assert ctypes.sizeof(st) == 8 * len(st._fields_)


def test_argument_block_entry_points_reject_null():
    from catfuse_amd import _hip
    assert _hip.lib().cf_conv_mfma_args(None) == INVALID
    assert _hip.lib().cf_conv_halo_pair_args(None) == INVALID
    assert _hip.lib().cf_conv_args_sizes(None) == INVALID
