"""CPU checks of the host side of the product (no GPU): the layer's workspace reservation against the inner delta
rule's needs, the cache-ring normalisation before a kernel writes into it, the compute-dtype rule, the product
core's conversion init against the closed form of ``HybridAttention.convert`` (``hibrit.py:211-240``), and the window
kernel's XCD item map."""
import ctypes
import math

import pytest
import torch

from heimdall_amd import _lib
from heimdall_amd._device import compute_dtype
from heimdall_amd.hibrit import BifrostCore, CoreConfig, _ring_to, n_archival


@pytest.fixture(scope="module")
def cpu_lib():
    if not _lib.LIB_PATH.exists():
        from heimdall_amd.build import build_library
        build_library()
    return _lib.load()


def _ws(lib, fn, *args):
    n = ctypes.c_size_t(0)
    assert getattr(lib, fn)(*args, ctypes.byref(n)) == 0
    return n.value


# The layer call runs the delta rule on B*Tq tokens, Tq = T - W from an empty cache and T otherwise, with the segment
# length chosen for B*T tokens; its reservation is the GDN layout of B*T tokens with that length.
CASES = [(1, 4, 4, 128, 512, 9728, 1), (1, 2, 8, 128, 1024, 10242, 1), (1, 2, 2, 64, 16, 20484, 0),
         (1, 4, 6, 256, 2048, 32768, 1), (3, 2, 3, 128, 16, 68, 1), (2, 4, 6, 256, 2048, 131072, 1)]


@pytest.mark.parametrize("B,G,R,D,W,T,bf16", CASES + [(b, g, r, d, w, t, dt) for b in (1, 2) for g, r in ((1, 1), (4, 6))
                                                     for d in (64, 256) for w in (64, 2048)
                                                     for t in (w + 1, 3 * w + 17, 40000) for dt in (0, 1)])
def test_layer_workspace_covers_inner_delta_rule(cpu_lib, B, G, R, D, W, T, bf16):
    L = cpu_lib.bf_gdn_segment_chunks(B * T, B, G, R, D)
    assert L > 0
    full = _ws(cpu_lib, "bf_gdn_workspace_size", B * T, B, G, R, D, bf16, L)
    for tq in (T, max(T - W, 0)):
        assert _ws(cpu_lib, "bf_gdn_workspace_size", B * tq, B, G, R, D, bf16, L) <= full
    layer = _ws(cpu_lib, "bf_layer_prefill_workspace_size", B, G, R, D, T, bf16)
    assert layer >= full


def test_ring_normalised_to_kernel_layouts():
    """A cache written by the reference holds the ring in the activations' dtype (and may be non-contiguous): before a
    kernel writes into it, ring_k / ring_v take the operand dtype and ring_km / ring_g / ring_beta fp32, densely."""
    st = dict(ring_k=torch.zeros(1, 2, 8, 4, dtype=torch.bfloat16), ring_v=torch.zeros(1, 2, 4, 8).transpose(2, 3),
              ring_km=torch.zeros(1, 8, 2, 4, dtype=torch.float16), ring_g=torch.zeros(1, 8, 2, dtype=torch.float64),
              ring_beta=torch.zeros(1, 8, 2), ring_pos=torch.full((8,), -1, dtype=torch.int32))
    _ring_to(st, torch.float32)
    assert st["ring_k"].dtype == st["ring_v"].dtype == torch.float32
    assert all(st[k].dtype == torch.float32 and st[k].is_contiguous() for k in ("ring_km", "ring_g", "ring_beta"))
    assert st["ring_v"].is_contiguous() and st["ring_pos"].dtype == torch.long
    _ring_to(st, torch.bfloat16)
    assert st["ring_k"].dtype == st["ring_v"].dtype == torch.bfloat16


def test_compute_dtype_rule():
    bf, f32, f16 = (torch.zeros(1, dtype=d) for d in (torch.bfloat16, torch.float32, torch.float16))
    assert compute_dtype(bf, bf) == torch.bfloat16
    assert compute_dtype(bf, f32) == torch.float32
    assert compute_dtype(f16, f16) == torch.float32          # fp16 is widened, never rounded to bf16
    with pytest.raises(_lib.BifrostError):
        compute_dtype(torch.zeros(1, dtype=torch.float64))


@pytest.mark.parametrize("hkv,archival", [(4, 1), (8, 2), (2, 0)])
def test_product_convert_closed_form(hkv, archival):
    """BifrostCore.convert: fq, fk identities, ab = 0, mix weight 0 and bias -2, mix_lse = 0, mem_scale = sqrt(D), the
    decay half-lives g = -ln2 / life at a = 0 with life = logspace(log10 W, 6, G), the first `archival` KV heads not
    decaying, dt = softplus(dt_bias) in [1e-3, 1e-1]."""
    torch.manual_seed(0)
    H, D, d, W = 2 * hkv, 32, 16, 512
    m = BifrostCore(CoreConfig(H, hkv, D, d))
    m.convert(W, 4, archival)
    assert m.window == W and m.sinks == 4
    assert torch.equal(m.fq, torch.eye(D).repeat(H, 1, 1)) and torch.equal(m.fk, torch.eye(D).repeat(hkv, 1, 1))
    assert not m.ab.weight.any() and not m.ab.bias.any() and not m.mix.weight.any()
    assert torch.equal(m.mix.bias, torch.full((H,), -2.0)) and not m.mix_lse.any()
    assert torch.allclose(m.mem_scale, torch.full((H,), math.sqrt(D)))
    dt = torch.nn.functional.softplus(m.dt_bias)
    assert ((dt >= 1e-3 * (1 - 1e-5)) & (dt <= 1e-1 * (1 + 1e-5))).all()
    g = -m.A_log.exp() * dt                                   # softplus(a + dt_bias) at a = 0
    life = torch.logspace(math.log10(W), 6.0, hkv)
    assert torch.allclose(-math.log(2) / g, life, rtol=1e-4)
    assert torch.equal(m.decay_mask, torch.tensor([0.0] * archival + [1.0] * (hkv - archival)))
    assert set(n for n, _ in m.named_parameters()) >= {"fq", "fk", "ab.weight", "mix.bias", "mix_lse", "mem_scale",
                                                         "A_log", "dt_bias"}


def test_n_archival():
    """hibrit.py:187-190: at least one archival head for the "long" init when a fraction is asked for."""
    assert n_archival(0.5, 4) == 2 and n_archival(0.1, 4) == 1 and n_archival(0.0, 4) == 0
    assert n_archival(0.1, 4, "mamba") == 0


def test_noalloc_decode_size_limit_without_gpu(cpu_lib):
    """The allocation-free decode entry point refuses a problem larger than its static scratch before any device
    call (placeholder pointers are never touched)."""
    n = ctypes.c_size_t(0)
    assert cpu_lib.bf_decode_workspace_size(256, 4, 8, 256, 8192, ctypes.byref(n)) == 0 and n.value > 16 << 20
    assert cpu_lib.bf_decode_fwd_noalloc(256, 4, 8, 256, 8192, 4, 100000, 1, 1, 1, *([256] * 12), 0, *([256] * 9),
                                         None) == -4


_WINMAP_CHECK = r"""
#include "bf_internal.h"
#include <cstdio>
#include <vector>
// Every work item of the bf16 window kernel comes from exactly one (XCD, dispatch slot), for every interleave f and
// rotation, and the slot count per XCD does not depend on f (the layer sizes its partial-row buffer without it).
int main() {
    long bad = 0, cases = 0;
    for (int B : {1, 2, 3, 5}) for (int G : {1, 2, 3, 4, 8}) for (int R : {1, 2, 6, 7})
    for (int T : {1, 100, 128, 129, 1000, 2048, 3000, 32768}) {
        const long per1 = bf::window_map_make(B, G, R, T, 1, 0).per;
        for (int f : {1, 2, 4, 8}) for (int rot : {0, 1, 31, 32, 1000}) {
            const bf::WinMap m = bf::window_map_make(B, G, R, T, f, rot);
            bad += m.per != per1;
            std::vector<int> seen(m.nrow * R, 0);
            for (int x = 0; x < 8; ++x)
                for (long k = 0; k < m.per; ++k) {
                    const long w = bf::window_item(m, x, k);
                    if (w < -1 || w >= m.nrow * R) ++bad;
                    else if (w >= 0) ++seen[w];
                }
            for (int c : seen) bad += c != 1;
            ++cases;
        }
    }
    printf("%ld %ld\n", cases, bad);
    return bad != 0;
}
"""


def test_window_item_map_is_a_bijection(tmp_path):
    """The window kernel's XCD item map (bf_internal.h window_item), compiled for the host with g++."""
    import shutil
    import subprocess
    from pathlib import Path
    gxx = shutil.which("g++")
    if gxx is None or not Path("/opt/rocm/include/hip/hip_runtime.h").exists():
        pytest.skip("g++ or the HIP headers are not available")
    src = tmp_path / "winmap.cpp"
    src.write_text(_WINMAP_CHECK)
    csrc = Path(__file__).resolve().parents[1] / "heimdall_amd" / "csrc"
    exe = tmp_path / "winmap"
    subprocess.run([gxx, "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{csrc}",
                    str(src), "-o", str(exe)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    cases, bad = map(int, out.stdout.split())
    assert out.returncode == 0 and bad == 0 and cases == 12800, out.stdout
