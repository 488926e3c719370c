"""Compile librngdpd.so (HIP, gfx950) and librngdpd_net.so (host-only tcp
transport) in place: ``python -m rngd_pd_amd.build``."""
import os
import subprocess
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_HERE)
SOURCES = ["handoff.hip", "attention.hip", "decode_step.hip", "wgemm.hip", "koni.hip",
           "staging.hip", "runtime.hip"]
OUT = os.path.join(_HERE, "librngdpd.so")
NET_SOURCES = ["net/tcpkv.cpp"]
NET_OUT = os.path.join(_HERE, "librngdpd_net.so")


def hipcc_command(out=OUT):
    return (["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
             "-shared", "-I", os.path.join(_ROOT, "include"),
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             # Leading scalar kernel arguments arrive preloaded in SGPRs, so a
             # kernel's first loads need not wait for a kernarg read.
             "-mllvm", "-amdgpu-kernarg-preload-count=16", "-o", out]
            + [os.path.join(_HERE, "csrc", s) for s in SOURCES])


def net_command(out=NET_OUT):
    """librngdpd_net.so: host code only (g++), no GPU runtime."""
    return (["g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-pthread", "-Wall",
             "-I", os.path.join(_ROOT, "include"), "-o", out]
            + [os.path.join(_HERE, "csrc", s) for s in NET_SOURCES])


def build_net(verbose=False):
    tmp = NET_OUT + ".tmp"
    r = subprocess.run(net_command(tmp), stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    if r.returncode != 0:
        raise RuntimeError("g++ failed:\n" + r.stdout)
    if verbose and r.stdout.strip():
        print(r.stdout)
    os.replace(tmp, NET_OUT)
    return NET_OUT


def build(verbose=False):
    build_net(verbose)
    tmp = OUT + ".tmp"
    r = subprocess.run(hipcc_command(tmp), stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    # The host pass warns that it does not know the packed-fp32 feature; nothing else is expected.
    noise = [ln for ln in r.stdout.splitlines() if "packed-fp32-ops" not in ln]
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(noise))
    if verbose and noise:
        print("\n".join(noise))
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
    sys.exit(0)
