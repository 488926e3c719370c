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
             "-mllvm", "-amdgpu-kernarg-preload-count=16",
             # Per-kernel register, scratch and occupancy report (checked below).
             "-Rpass-analysis=kernel-resource-usage", "-o", out]
            + [os.path.join(_HERE, "csrc", s) for s in SOURCES])


# Kernels of the handoff and attention paths: a lane's state must fit its
# registers. A build in which any of them needs scratch (private) memory is
# refused: a spill there once cost a serving step 2 ms unnoticed by every
# correctness test. The decode-step GEMMs for more than 16 streams with wide
# column groups do spill and are allowed (wgemm_kernel is not listed).
NO_SCRATCH = ("decode_attn_kernel", "merge_kernel", "pack_kernel", "scatter_kernel",
              "gather_kernel", "koni_scatter_kernel", "koni_gather_kernel")


def resource_report(text):
    """{mangled kernel name: {field: value}} from -Rpass-analysis=kernel-resource-usage."""
    out, cur = {}, None
    for ln in text.splitlines():
        if "remark:" not in ln or "kernel-resource-usage" not in ln:
            continue
        body = ln.split("remark:", 1)[1].rsplit("[-Rpass-analysis", 1)[0].strip()
        key, _, val = body.partition(":")
        if key == "Function Name":
            cur = out.setdefault(val.strip(), {})
        elif cur is not None:
            cur[key.strip()] = val.strip()
    return out


def scratch_kernels(report, names=NO_SCRATCH):
    """(kernel, bytes per lane) of the listed kernels that use scratch memory."""
    bad = []
    for fn, fields in report.items():
        if any(n in fn for n in names) and int(fields.get("ScratchSize [bytes/lane]", "0")) > 0:
            bad.append((fn, int(fields["ScratchSize [bytes/lane]"])))
    return bad


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
    # The host pass warns that it does not know the packed-fp32 feature, and
    # the resource remarks are read below; nothing else is expected.
    noise = [ln for ln in r.stdout.splitlines()
             if "packed-fp32-ops" not in ln and "kernel-resource-usage" not in ln
             and not ln.lstrip().startswith(("|", "^")) and not ln.strip()[:1].isdigit()]
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(noise))
    bad = scratch_kernels(resource_report(r.stdout))
    if bad:
        os.remove(tmp)
        raise RuntimeError("kernels that must keep their state in registers use scratch memory: "
                           + ", ".join(f"{fn} ({n} bytes/lane)" for fn, n in bad))
    if verbose and noise:
        print("\n".join(noise))
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
    sys.exit(0)
