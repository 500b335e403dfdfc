"""The on-disk cache of generated code objects is keyed by what decides them.

``native.rtc_cache_key`` hashes the architecture, the compiler fingerprint
(``ye3t_hip_rtc_fingerprint``: hipRTC version, the options of
``ye3t_hip_rtc_compile`` and the ABI version) and the source, so a library
built with other options, another hipRTC or another ABI never loads a stale
code object.  hipRTC runs on the host, so these tests need no GPU.
"""

import os

from ye3t_amd.runtime import native

SRC = 'extern "C" __global__ void k(double* x) { x[threadIdx.x] *= 2.0; }'


def test_fingerprint_names_version_options_and_abi():
    fp = native.rtc_fingerprint()
    assert fp.startswith("hiprtc ")
    assert "-O3" in fp and "-packed-fp32-ops" in fp
    assert fp.endswith(f"abi {native.ABI_VERSION}")


def test_key_changes_with_each_input(monkeypatch):
    base = native.rtc_cache_key(SRC)
    assert base == native.rtc_cache_key(SRC)
    assert native.rtc_cache_key(SRC + " ") != base
    assert native.rtc_cache_key(SRC, arch="gfx942") != base
    real = native.rtc_fingerprint()
    for other in (real.replace("-O3", "-O2"), real.replace(f"abi {native.ABI_VERSION}", "abi 1"),
                  "hiprtc 0.0" + real[real.index(" |"):]):
        monkeypatch.setattr(native, "rtc_fingerprint", lambda other=other: other)
        assert native.rtc_cache_key(SRC) != base


def test_compile_lands_under_the_key(tmp_path, monkeypatch):
    monkeypatch.setenv("YE3T_AMD_JIT_CACHE", str(tmp_path))
    blob = native.rtc_compile(SRC, name="k.hip")
    path = tmp_path / (native.rtc_cache_key(SRC) + ".co")
    assert path.exists() and path.read_bytes() == blob
    assert blob[:4] == b"\x7fELF"
    assert len(os.listdir(tmp_path)) == 1
