"""The committed golden fixtures (tests/golden/*.npz): the CPU oracle regenerates
every one of them exactly (CPU), and the GPU kernels reproduce them within the
gates, or byte for byte for the store (GPU)."""

import glob
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FILES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixtures_exist():
    assert len(FILES) >= 8


@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f)[:-4] for f in FILES])
def test_oracle_regenerates_fixture(path):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    name = os.path.basename(path)[:-4]
    fresh = next(dict([c()]) for c in mg.CASES if c()[0] == name)[name]
    stored = load(path)
    assert set(stored) == set(fresh)
    for key, val in fresh.items():
        np.testing.assert_array_equal(np.asarray(val), stored[key], err_msg=key)


def _torch_bits(arr, dtype, device):
    import torch

    if dtype == "bf16":
        return torch.from_numpy(arr.astype(np.uint16).view(np.int16)).view(torch.bfloat16).to(device)
    return torch.from_numpy(np.ascontiguousarray(arr, np.float32)).to(device)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f)[:-4] for f in FILES])
def test_gpu_matches_fixture(cuda, path):
    import torch

    import cpu_attention as C
    from helpers import assert_close, cache_words

    f = load(path)
    dtype = str(f["dtype"])
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    if str(f["kind"]) == "flash":
        q, k, v = (_torch_bits(f[x], dtype, cuda) for x in ("q", "k", "v"))
        out = C.flash_attn_func(q, k, v, softmax_scale=float(f["scale"]), causal=bool(f["causal"]))
        assert_close(out, f["out"], tdt, paged=False)
    elif str(f["kind"]) == "decode":
        kc = torch.from_numpy(f["kc"].view(np.int32)).to(cuda).view(tdt)
        vc = torch.from_numpy(f["vc"].view(np.int32)).to(cuda).view(tdt)
        nb, h = f["kc"].shape[:2]
        page = int(f["page"])
        d = f["q"].shape[-1]
        kc, vc = kc.view(nb, h, page, d), vc.view(nb, h, page, d)
        q = _torch_bits(f["q"], dtype, cuda)[:, None]
        out = C.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=torch.from_numpy(f["lens"]).to(cuda),
                                        page_table=torch.from_numpy(f["table"]).to(cuda),
                                        softmax_scale=float(f["scale"]))
        assert_close(out[:, 0], f["out"], tdt, paged=True)
    else:
        page = int(f["page"])
        nb, h = f["kc"].shape[:2]
        d = f["key"].shape[-1]
        kc = torch.zeros(nb, h, page, d, dtype=tdt, device=cuda)
        vc = torch.zeros_like(kc)
        C.reshape_and_cache(_torch_bits(f["key"], dtype, cuda), _torch_bits(f["value"], dtype, cuda),
                            kc, vc, torch.from_numpy(f["slots"]).to(cuda))
        np.testing.assert_array_equal(cache_words(kc), f["kc"])
        np.testing.assert_array_equal(cache_words(vc), f["vc"])
