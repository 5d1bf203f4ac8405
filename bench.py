"""Benchmark of the KAD-Conv inference hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-ops] [--no-cpu] [--no-kadcnet]
                    [--per-op-only] [--kadcnet-only]

Step = one fused KADConv(256) forward on x [8, 256, 100, 100] fp16 (BASELINE
config 2's metric shape), inputs resident in HBM, weights random from a seed
(synthetic; no checkpoint exists offline).  The forward is captured once in a
HIP graph and replayed (the reference protocol, KAD-CNet/inference/benchmark_s.py:9-25):
W warm-up replays, then 3 trials of K replays timed between events; the
median trial is reported.

Printed: one JSON line with
  value / ms_per_step      microseconds per forward (lower is better), median of 3 trials;
  roofline                 the dominant kernel (branch-0 DCN) timed alone with
                           events on its launch stream: algorithmic FLOPs / duration
                           against the fp16 dense MFMA peak;
  forward_roofline         BASELINE's derived floor for the whole forward (10.33 us)
                           over the measured time;
  cpu_baseline             the oracle's fp32 CPU restatement of the reference forward
                           (plain PyTorch ops), same shape, on this host's cores;
  stages_us                per-stage event timings of one forward;
  kadcnet_s_img_per_s      BASELINE config 5: KAD-CNet-S forward, batch 16, 800 x 800, fp16
                           (details and its CPU baseline under kadcnet_s);
  per_op                   configs 2-4 (DSC, KADDown, 1x1+SiLU, SE): GPU us, floor, and the
                           oracle's fp32 CPU us of the same workload;
  config1                  config 1: KADConv(64) / DSC(64) at [1, 64, 80, 80] fp32, the plain
                           CPU forward, the oracle's CPU time and the GPU fast path.
"""
import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, 'kad-conv_amd'))
sys.path.insert(0, ROOT)

PEAK_MFMA_F16 = 2516.6e12   # dense fp16/bf16 MFMA, 256 CU x 2.4 GHz x 4096 flop/clk
PEAK_HBM = 8.0e12
FORWARD_FLOOR_US = 10.33    # max(MFMA, HBM) floor for KADConv(256) at [8,256,100,100] fp16


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def time_graph(fn, steps, warmup, trials=3):
    """Capture fn in a graph, replay it `warmup` times, then time `trials` runs of
    `steps` replays between events (the reference protocol,
    KAD-CNet/inference/benchmark_s.py:9-25).  Returns (median us per replay,
    [us per replay of each trial], graph)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    vals = []
    for _ in range(trials):
        a, b = _events()
        a.record()
        for _ in range(steps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        vals.append(a.elapsed_time(b) * 1e3 / steps)
    return sorted(vals)[len(vals) // 2], vals, g


def time_eager(fn, steps, warmup=3):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = _events()
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / steps


def metric_state(dim, seed=0):
    """Synthetic weights of the metric's layer (kadconv.synthetic.make_metric_kadconv_state)."""
    from kadconv import synthetic as S
    return S.make_metric_kadconv_state(dim, seed=seed)


def build_kadconv(dim, dtype, seed=0):
    import kadconv
    m = kadconv.KADConv(dim)
    m.load_state_dict(metric_state(dim, seed), strict=False)
    return m.to('cuda', dtype).eval()


def dsc_flops(n, h, w, c):
    """Algorithmic flops of one DSC launch: deformable conv c -> c plus conv_offset c -> 18 (3x3)."""
    return 2.0 * n * h * w * 9 * c * (c + 18)


def cpu_baseline(shape, runs=5, warmup=2):
    """The oracle's fp32 restatement of the reference plain-PyTorch forward
    (oracle/kadconv_oracle.py:kadconv_forward), timed on this host."""
    from oracle import kadconv_oracle as O
    threads = len(os.sched_getaffinity(0))
    sd = metric_state(shape[1])
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(0))
    sec = _cpu_time(lambda: O.kadconv_forward(sd, x), runs=runs, warmup=warmup)
    return {'value': sec * 1e6, 'unit': 'us', 'cores': torch.get_num_threads(), 'kind': 'port',
            'sample': f'full workload x{list(shape)} fp32, median of {runs} after {warmup} warm-up runs '
                      f'(os.cpu_count={os.cpu_count()}, affinity={threads}, cpu="{_cpu_model()}")'}


# KAD-CNet-S DSC(c, c) shapes at 800 x 800: c in {12, 10, 10} at {100, 50, 25}^2, {16, 16, 16} at
# {50, 25, 12}^2, {22, 21, 21} at {25, 12, 6}^2
KADCNET_DSC = [(12, 100), (10, 50), (10, 25), (16, 50), (16, 25), (16, 12), (22, 25), (21, 12), (21, 6)]


def per_op_workloads():
    """The other BASELINE configs as (name, launch, floor_us) with seeded inputs and weights."""
    import kadconv
    from kadconv import synthetic as S
    out = []
    g = torch.Generator().manual_seed(0)
    dt = torch.float16
    # config 2: DSC(C, C) at the neck scales
    for C, H in [(128, 100), (256, 50), (512, 25)]:
        d = kadconv.DSC(C, C)
        d.load_state_dict(S.make_dsc_state(C, C, seed=C, offset_std_px=2.0), strict=False)
        d = d.to('cuda', dt).eval()
        kadconv.enable_fast_inference(d)
        x = torch.randn(8, C, H, H, generator=g).to('cuda', dt)
        fl = 8 * H * H * (2 * 9 * C * C + 2 * 9 * 18 * C + 2 * 9 * C + 44 * C)
        by = 2 * 8 * C * H * H * 2 + 2 * (9 * C * C + 162 * C + 9 * C)
        out.append((f'dsc_{C}x{H}', lambda d=d, x=x: d(x), max(fl / PEAK_MFMA_F16, by / PEAK_HBM) * 1e6))
    # config 3: KADDown [8,256,100,100] -> [8,512,50,50]
    m = kadconv.KADDown(256, 512)
    m.load_state_dict(S.make_kaddown_state(256, 512))
    m = m.to('cuda', dt).eval()
    x = torch.randn(8, 256, 100, 100, generator=g).to('cuda', dt)
    out.append(('kaddown_256to512_100', lambda m=m, x=x: m(x), max(6.86e9 / PEAK_MFMA_F16, 61.44e6 / PEAK_HBM) * 1e6))
    # config 4a: 1x1 conv + SiLU [16,512,50,50]
    m = kadconv.Conv1x1SiLU(512, 512)
    with torch.no_grad():
        m.conv.weight.normal_(0, 0.02)
        m.conv.bias.normal_(0, 0.02)
    m = m.to('cuda', dt).eval()
    x = torch.randn(16, 512, 50, 50, generator=g).to('cuda', dt)
    out.append(('conv1x1_silu_512_50', lambda m=m, x=x: m(x), max(20.97e9 / PEAK_MFMA_F16, 82.44e6 / PEAK_HBM) * 1e6))
    # config 4b: SE [16,1024,25,25], r=16
    m = kadconv.SqueezeExcitation(1024, reduction=16).to('cuda', dt).eval()
    x = torch.randn(16, 1024, 25, 25, generator=g).to('cuda', dt)
    out.append(('se_1024_25', lambda m=m, x=x: m(x), 40.96e6 / PEAK_HBM * 1e6))
    # config 5's DSC(c, c) shapes (KAD-CNet-S, bs16 at 800 x 800), channels-last as in the network
    for C, H in KADCNET_DSC:
        d = kadconv.DSC(C, C)
        d.load_state_dict(S.make_dsc_state(C, C, seed=C * 7 + H, offset_std_px=2.0), strict=False)
        d = d.to('cuda', dt).eval()
        kadconv.enable_fast_inference(d)
        x = torch.randn(16, C, H, H, generator=g).to('cuda', dt).contiguous(memory_format=torch.channels_last)
        fl = 16 * H * H * (2 * 9 * C * C + 2 * 9 * 18 * C + 2 * 9 * C + 44 * C)
        by = 2 * 16 * C * H * H * 2 + 2 * (9 * C * C + 162 * C + 9 * C)
        out.append((f'kadcnet_dsc_{C}x{H}', lambda d=d, x=x: d(x), max(fl / PEAK_MFMA_F16, by / PEAK_HBM) * 1e6))
    return out


def _cpu_model():
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return ''


def _cpu_time(fn, runs=5, warmup=2):
    """Median seconds of fn() on this host's cores (all threads of the affinity set)."""
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    ts = []
    with torch.no_grad():
        for i in range(warmup + runs):
            t0 = time.perf_counter()
            fn()
            if i >= warmup:
                ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def per_op_cpu():
    """The oracle's fp32 CPU restatement of each per-op workload (the reference's plain
    PyTorch path, torchvision's deform_conv2d restated), same shapes and seeds as
    per_op_workloads(): name -> median us."""
    from kadconv import synthetic as S
    from oracle import kadconv_oracle as O
    out = {}
    g = torch.Generator().manual_seed(0)
    for C, H in [(128, 100), (256, 50), (512, 25)]:
        sd = S.make_dsc_state(C, C, seed=C, offset_std_px=2.0)
        x = torch.randn(8, C, H, H, generator=g)
        out[f'dsc_{C}x{H}'] = _cpu_time(lambda sd=sd, x=x: O.dsc_forward(sd, '', x)) * 1e6
    sd = S.make_kaddown_state(256, 512)
    x = torch.randn(8, 256, 100, 100, generator=g)
    out['kaddown_256to512_100'] = _cpu_time(lambda: O.kaddown_forward(sd, x)) * 1e6
    w, b = torch.randn(512, 512) * 0.02, torch.randn(512) * 0.02
    x = torch.randn(16, 512, 50, 50, generator=g)
    out['conv1x1_silu_512_50'] = _cpu_time(lambda: O.conv1x1_silu(x, w, b)) * 1e6
    se = torch.nn.Sequential(torch.nn.Linear(1024, 64), torch.nn.ReLU(), torch.nn.Linear(64, 1024))
    p = [t.detach() for t in (se[0].weight, se[0].bias, se[2].weight, se[2].bias)]
    x = torch.randn(16, 1024, 25, 25, generator=g)
    out['se_1024_25'] = _cpu_time(lambda: O.se_forward(x, *p)) * 1e6
    for C, H in KADCNET_DSC:
        sd = S.make_dsc_state(C, C, seed=C * 7 + H, offset_std_px=2.0)
        x = torch.randn(16, C, H, H, generator=g)
        out[f'kadcnet_dsc_{C}x{H}'] = _cpu_time(lambda sd=sd, x=x: O.dsc_forward(sd, '', x)) * 1e6
    return out


PER_OP_BATCH = 10  # calls per graph for the amortised figure


def per_op(steps, warmup, cpu=True):
    """The other BASELINE configs, graph-timed (median of 3 trials, us per call) with
    their floors, and the oracle's fp32 CPU time of the same workload.  `us` replays a graph
    of one call (the reference protocol); `us_graph10` replays a graph of PER_OP_BATCH calls
    of the same op on the same input and divides by PER_OP_BATCH: the replay's fixed cost (about
    10 us per replay here, GPU-side, plus a host cost of 15-20 us per replay that bounds graphs
    shorter than that) is then shared, so for the short ops it is the figure that measures the
    kernels."""
    res = {}
    for name, fn, floor in per_op_workloads():
        us, trials, _ = time_graph(fn, steps, warmup)
        us10, _, _ = time_graph(lambda fn=fn: [fn() for _ in range(PER_OP_BATCH)], max(steps // PER_OP_BATCH, 5),
                                max(warmup // PER_OP_BATCH, 2))
        us10 /= PER_OP_BATCH
        res[name] = {'us': round(us, 2), 'trials_us': [round(t, 2) for t in trials], 'floor_us': round(floor, 2),
                     'frac': round(floor / us, 4), 'us_graph10': round(us10, 2), 'frac_graph10': round(floor / us10, 4)}
    if cpu:
        for name, us in per_op_cpu().items():
            res[name]['cpu_us'] = round(us, 1)
    return res


def config1(steps, warmup, cpu=True):
    """KADConv(64) and DSC(64) on [1, 64, 80, 80] fp32, every weight
    kaiming-uniform from seed 0.  Reported: the product's plain CPU forward (the
    plumbing the config asks for), the oracle's (the reference's plain path restated),
    and the fast HIP forward on the GPU for scale."""
    import kadconv
    from kadconv import synthetic as S
    from oracle import kadconv_oracle as O
    out = {}
    x = torch.randn(1, 64, 80, 80, generator=torch.Generator().manual_seed(0))
    for name, mk, sdf, ref in [
            ('kadconv_64_80_f32', lambda: kadconv.KADConv(64), lambda: S.make_kadconv_state(64, seed=0),
             lambda sd: O.kadconv_forward(sd, x)),
            ('dsc_64_80_f32', lambda: kadconv.DSC(64, 64), lambda: S.make_dsc_state(64, 64, seed=0),
             lambda sd: O.dsc_forward(sd, '', x))]:
        m = mk()
        sd = sdf()
        m.load_state_dict(sd, strict=False)
        m.eval()
        row = {}
        if cpu:
            row['cpu_plain_us'] = round(_cpu_time(lambda: m(x)) * 1e6, 1)
            row['cpu_us'] = round(_cpu_time(lambda: ref(sd)) * 1e6, 1)
        md = m.to('cuda')
        kadconv.enable_fast_inference(md)
        xd = x.cuda()
        with torch.no_grad():
            us, _, _ = time_graph(lambda: md(xd), steps, warmup)
        row['us'] = round(us, 2)
        out[name] = row
    return out


def kadcnet_flops(hw=800):
    """Multiply-add FLOPs (2 per MAC) of one KAD-CNet-S image at hw x hw, from forward hooks on
    the fused model's plain CPU forward of one hw x hw image (about 2 s): every Conv2d (groups
    honoured; the LCSA strip convs at full resolution, as the kernels form them), every Linear,
    and each DSC's deformable 3 x 3 (2 * 9 * Cin per output value).  Element-wise work
    (activations, pooling, resize, merges, decode) is not counted."""
    import kadcnet
    import kadconv
    model = kadcnet.build_kadcnet_s(seed=0).fuse().eval()
    tot = [0]

    def conv(m, i, o):
        tot[0] += 2 * (m.in_channels // m.groups) * m.kernel_size[0] * m.kernel_size[1] * o.numel()

    def lin(m, i, o):
        tot[0] += 2 * m.in_features * o.numel()

    def dsc(m, i, o):
        tot[0] += 2 * 9 * m.weight.shape[1] * o.numel()
    hooks = []
    for mod in model.modules():
        if isinstance(mod, torch.nn.Conv2d):
            hooks.append(mod.register_forward_hook(conv))
        elif isinstance(mod, torch.nn.Linear):
            hooks.append(mod.register_forward_hook(lin))
        elif isinstance(mod, kadconv.DSC):
            hooks.append(mod.register_forward_hook(dsc))
    with torch.no_grad():
        model(torch.zeros(1, 3, hw, hw))
    for h in hooks:
        h.remove()
    return tot[0]


def kadcnet_s(iterations, warmup, cpu=True, batch=16, hw=800):
    """the whole KAD-CNet-S forward (fused model, random init from
    seed 0, kadcnet.build_kadcnet_s), batch 16, 3 x 800 x 800 ~U[0, 1], fp16,
    model forward only (no NMS), HIP-graph replay, median of 3 trials
    (KAD-CNet/inference/benchmark_s.py:9-25).  CPU baseline: the oracle's fp32
    restatement on a bounded sample of 2 images of the batch (img/s)."""
    import kadcnet
    model = kadcnet.build_kadcnet_s(seed=0).fuse()
    m = model.to('cuda', torch.float16).eval()
    kadcnet.enable_fast_inference(m)
    x = torch.rand(batch, 3, hw, hw, generator=torch.Generator().manual_seed(0))
    xd = x.to('cuda', torch.float16)
    with torch.no_grad():
        us, trials, _ = time_graph(lambda: m(xd), iterations, warmup)
    out = {'img_per_s': round(batch / (us * 1e-6), 1), 'ms_per_batch': round(us / 1e3, 3),
           'trials_ms': [round(t / 1e3, 3) for t in trials], 'batch': batch, 'hw': [hw, hw], 'dtype': 'f16',
           'iterations': iterations, 'warmup': warmup}
    fl = kadcnet_flops(hw)
    out['gflop_per_img'] = round(fl / 1e9, 2)
    out['tflop_per_s'] = round(fl * batch / (us * 1e-6) / 1e12, 1)
    out['mfma_frac'] = round(fl * batch / (us * 1e-6) / PEAK_MFMA_F16, 4)
    out['flops_note'] = ('2 x MACs of every convolution, Linear and deformable 3 x 3 (kadcnet_flops), per image; '
                         'mfma_frac = achieved FLOP/s over the 2516.6 TFLOP/s dense fp16 peak')
    if cpu:
        from oracle import kadcnet_oracle as KO
        sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
        xs = x[:2].float()
        sec = _cpu_time(lambda: KO.kadcnet_forward(sd, kadcnet.DIOR_S_BASE, xs), runs=3, warmup=1)
        out['cpu_baseline'] = {'value': round(2 / sec, 3), 'unit': 'img/s', 'cores': torch.get_num_threads(),
                               'kind': 'port', 'sample': f'2 of the 16 images, fp32, median of 3 after 1 warm-up '
                                                         f'(cpu="{_cpu_model()}")'}
    return out


TRAFFIC_FILE = os.path.join(ROOT, 'profiles', 'dsc0_traffic.json')
PROBE_COPY_BYTES = 64 << 20


def traffic_probe():
    """A short program for the two rocprofv3 --pmc passes (FETCH_SIZE, then
    WRITE_SIZE): a plain 64 MiB device copy (the scale reference) and the
    dominant kernel (branch-0 DSC of the metric's forward), 5 dispatches each."""
    import kadconv
    m = build_kadconv(256, torch.float16)
    kadconv.enable_fast_inference(m)
    x = torch.randn(8, 256, 100, 100, generator=torch.Generator().manual_seed(0)).to('cuda', torch.float16)
    with torch.no_grad():
        st, _ = m._kad_plan.stages(x)
        for _, fn in st:
            fn()
        dsc0 = dict(st).get('dsc') or dict(st)['dsc0']
        a = torch.empty(PROBE_COPY_BYTES, dtype=torch.uint8, device='cuda')
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        for _ in range(5):
            dsc0()
        torch.cuda.synchronize()
    print(json.dumps({'probe': 'done', 'copy_bytes': PROBE_COPY_BYTES}), flush=True)


def counters_probe():
    """A short program for the per-kernel counter table (rocprofv3 --pmc passes and
    a kernel trace): every stage of the metric's forward, eagerly, then each per-op
    workload, 3 times each, then the 64 MiB copy that scales FETCH_SIZE / WRITE_SIZE."""
    import kadconv
    m = build_kadconv(256, torch.float16)
    kadconv.enable_fast_inference(m)
    x = torch.randn(8, 256, 100, 100, generator=torch.Generator().manual_seed(0)).to('cuda', torch.float16)
    with torch.no_grad():
        st, _ = m._kad_plan.stages(x)
        for _ in range(3):
            for _, fn in st:
                fn()
                torch.cuda.synchronize()
        for _, fn, _ in per_op_workloads():
            for _ in range(3):
                fn()
                torch.cuda.synchronize()
        a = torch.empty(PROBE_COPY_BYTES, dtype=torch.uint8, device='cuda')
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
    print(json.dumps({'probe': 'done', 'copy_bytes': PROBE_COPY_BYTES}), flush=True)


def counters_probe_net():
    """A short program for the KAD-CNet-S counter table: two eager forwards of config 5 (fused
    model, bs16, 3 x 800 x 800 fp16; the first builds the plan), then the 64 MiB copy."""
    import kadcnet
    m = kadcnet.build_kadcnet_s(seed=0).fuse().to('cuda', torch.float16).eval()
    kadcnet.enable_fast_inference(m)
    x = torch.rand(16, 3, 800, 800, generator=torch.Generator().manual_seed(0)).to('cuda', torch.float16)
    with torch.no_grad():
        for _ in range(3):
            m(x)
            torch.cuda.synchronize()
            torch.cuda._sleep(1000)  # a spin kernel between forwards: the summary splits the dispatches there
            torch.cuda.synchronize()
        a = torch.empty(PROBE_COPY_BYTES, dtype=torch.uint8, device='cuda')
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
    print(json.dumps({'probe': 'done', 'copy_bytes': PROBE_COPY_BYTES, 'forwards': 3}), flush=True)


def counters_net_from(trace_csv, fetch_csv, write_csv, sq_csv, forwards=3, top=12):
    """Per-kernel table of the KAD-CNet-S forward from counters_probe_net(): each kernel's
    dispatches of forwards 2 .. `forwards` (the first builds the plan) summed and divided by their
    number (us, MB read / written per forward); MFMA busy over the kernel's own cycles (sum of
    SQ_VALU_MFMA_BUSY_CYCLES over the sum of GRBM_GUI_ACTIVE / 8 x 1024 SIMDs)."""
    import collections
    import csv

    def rows_of(path, counter=None):
        d = collections.defaultdict(list)
        for r in csv.DictReader(open(path)):
            if counter is None or r['Counter_Name'] == counter:
                d[int(r['Dispatch_Id'])].append(r)
        return [d[k] for k in sorted(d)]

    def tail(disp):  # dispatches of forwards 2 .. forwards: between the first and the last spin kernel
        marks = [i for i, rs in enumerate(disp) if 'spin_kernel' in rs[0]['Kernel_Name']]
        return [rs for rs in disp[marks[0] + 1:marks[-1]] if 'spin_kernel' not in rs[0]['Kernel_Name']]
    tr = rows_of(trace_csv)
    f, w, sq = rows_of(fetch_csv, 'FETCH_SIZE'), rows_of(write_csv, 'WRITE_SIZE'), rows_of(sq_csv)
    cf = [float(rs[0]['Counter_Value']) for rs in f if 'copyBuffer' in rs[0]['Kernel_Name']][-3:]
    cw = [float(rs[0]['Counter_Value']) for rs in w if 'copyBuffer' in rs[0]['Kernel_Name']][-3:]
    sf = PROBE_COPY_BYTES / (sorted(cf)[1] * 1024.0)   # the three 64 MiB copies at the end
    sw = PROBE_COPY_BYTES / (sorted(cw)[1] * 1024.0)
    nf = forwards - 1
    agg = collections.defaultdict(lambda: [0, 0.0, 0.0, 0.0, 0.0, 0.0])
    for rs in tail(tr):
        r = rs[0]
        a = agg[r['Kernel_Name']]
        a[0] += 1
        a[1] += (int(r['End_Timestamp']) - int(r['Start_Timestamp'])) / 1e3
    for rs in tail(f):
        agg[rs[0]['Kernel_Name']][2] += float(rs[0]['Counter_Value']) * 1024.0 * sf
    for rs in tail(w):
        agg[rs[0]['Kernel_Name']][3] += float(rs[0]['Counter_Value']) * 1024.0 * sw
    for rs in tail(sq):
        v = {r['Counter_Name']: float(r['Counter_Value']) for r in rs}
        a = agg[rs[0]['Kernel_Name']]
        a[4] += v.get('SQ_VALU_MFMA_BUSY_CYCLES', 0.0)
        a[5] += v.get('GRBM_GUI_ACTIVE', 0.0) / 8.0 * 1024.0
    tot_us = sum(a[1] for a in agg.values()) / nf
    tot_rd = sum(a[2] for a in agg.values()) / nf
    tot_wr = sum(a[3] for a in agg.values()) / nf
    lines = ['| kernel | launches / forward | us / forward | share | read MB | write MB | GB/s | MFMA busy |',
             '|---|---|---|---|---|---|---|---|']
    for name, a in sorted(agg.items(), key=lambda kv: -kv[1][1])[:top]:
        us, rd, wr = a[1] / nf, a[2] / nf / 1e6, a[3] / nf / 1e6
        short = name if len(name) < 70 else name[:67] + '...'
        busy = a[4] / a[5] if a[5] else float('nan')
        lines.append(f'| `{short}` | {a[0] / nf:.0f} | {us:.1f} | {100 * us / tot_us:.1f}% | {rd:.1f} | {wr:.1f} | '
                     f'{(rd + wr) * 1e6 / (us * 1e-6) / 1e9:.0f} | {100 * busy:.1f}% |')
    tot_mf = sum(a[4] for a in agg.values())
    tot_cy = sum(a[5] for a in agg.values())
    lines.append(f'| all {len(agg)} kernels | {sum(a[0] for a in agg.values()) / nf:.0f} | {tot_us:.1f} | 100% | '
                 f'{tot_rd / 1e6:.1f} | {tot_wr / 1e6:.1f} | {(tot_rd + tot_wr) / (tot_us * 1e-6) / 1e9:.0f} | '
                 f'{100 * tot_mf / tot_cy:.1f}% |')
    print('\n'.join(lines))
    print(json.dumps({'fetch_scale': sf, 'write_scale': sw, 'forwards_counted': nf}))


def traffic_from(fetch_csv, write_csv):
    """HBM bytes per launch of the dominant kernel from the two --pmc runs of
    traffic_probe(): each counter (KiB per dispatch) is scaled by what it reads
    for the 64 MiB copy, whose true traffic is 64 MiB read + 64 MiB written."""
    import csv
    import statistics

    def per_kernel(path, counter):
        # dispatches of the largest grid of each kind: the 64 MiB copy and the branch-0 DSC
        rows = {'copy': [], 'dsc0': []}
        for r in csv.DictReader(open(path)):
            if r['Counter_Name'] != counter:
                continue
            name = r['Kernel_Name']
            grid = int(r.get('Grid_Size') or r.get('Grid_Size_X') or 0)
            kind = 'dsc0' if ('dcn_fwd_kernel' in name or 'dcn_group_kernel' in name) else \
                'copy' if 'copy' in name.lower() else None
            if kind:
                rows[kind].append((grid, float(r['Counter_Value'])))
        out = {}
        for kind, v in rows.items():
            gmax = max(g for g, _ in v)
            out[kind] = statistics.median([x for g, x in v if g == gmax])
        return out

    f, w = per_kernel(fetch_csv, 'FETCH_SIZE'), per_kernel(write_csv, 'WRITE_SIZE')
    sf = PROBE_COPY_BYTES / (f['copy'] * 1024.0)
    sw = PROBE_COPY_BYTES / (w['copy'] * 1024.0)
    rd, wr = f['dsc0'] * 1024.0 * sf, w['dsc0'] * 1024.0 * sw
    out = {'kernel': 'dcn_fwd_kernel<half,half,6,FUSED> branch-0 DSC, [8,86,100,100] fp16',
           'fetch_kib_raw': f['dsc0'], 'write_kib_raw': w['dsc0'],
           'copy_fetch_kib_raw': f['copy'], 'copy_write_kib_raw': w['copy'],
           'fetch_scale': sf, 'write_scale': sw,
           'read_bytes': rd, 'write_bytes': wr, 'bytes_per_launch': rd + wr}
    json.dump(out, open(TRAFFIC_FILE, 'w'), indent=1)
    print(json.dumps(out))


COUNTERS_FILE = os.path.join(ROOT, 'profiles', 'kernel_counters.md')


def counters_from(trace_csv, fetch_csv, write_csv, sq_csv):
    """Per-kernel table from one kernel trace and three --pmc runs of counters_probe().
    HBM bytes: FETCH_SIZE / WRITE_SIZE (KiB per dispatch) scaled by their reading for
    the 64 MiB copy (true: 64 MiB read + 64 MiB written).  MFMA busy: summed
    SQ_VALU_MFMA_BUSY_CYCLES over all 1024 SIMDs' cycles, the latter from
    GRBM_GUI_ACTIVE (which reads one count per XCD, 8 per dispatch-cycle)."""
    import collections
    import csv
    import statistics

    def pmc(path):
        d = collections.defaultdict(lambda: collections.defaultdict(list))
        for r in csv.DictReader(open(path)):
            d[(r['Kernel_Name'], int(r['Grid_Size']))][r['Counter_Name']].append(float(r['Counter_Value']))
        return d
    f, w, sq = pmc(fetch_csv), pmc(write_csv), pmc(sq_csv)
    dur = collections.defaultdict(list)
    for r in csv.DictReader(open(trace_csv)):
        g = int(r['Grid_Size_X']) * int(r['Grid_Size_Y']) * int(r['Grid_Size_Z'])
        dur[(r['Kernel_Name'], g)].append((int(r['End_Timestamp']) - int(r['Start_Timestamp'])) / 1e3)
    copy = [k for k in f if 'copyBuffer' in k[0]]
    ck = max(copy, key=lambda k: k[1])
    sf = PROBE_COPY_BYTES / (statistics.median(f[ck]['FETCH_SIZE']) * 1024.0)
    sw = PROBE_COPY_BYTES / (statistics.median(w[ck]['WRITE_SIZE']) * 1024.0)
    rows = []
    for k in f:
        name, grid = k
        if not (name.startswith(('_ZN3kad', 'kad::', 'void kad::')) or 'scale_residual' in name) or 'pack_kernel' in name \
                or k not in dur:
            continue
        us = statistics.median(dur[k])
        rd = statistics.median(f[k]['FETCH_SIZE']) * 1024.0 * sf
        wr = statistics.median(w[k]['WRITE_SIZE']) * 1024.0 * sw if k in w else float('nan')
        mf = statistics.median(sq[k]['SQ_VALU_MFMA_BUSY_CYCLES']) if k in sq else 0.0
        gr = statistics.median(sq[k]['GRBM_GUI_ACTIVE']) if k in sq else float('nan')
        busy = mf / (gr / 8.0 * 1024.0) if gr == gr and gr > 0 else float('nan')
        gbs = (rd + wr) / (us * 1e-6) / 1e9
        rows.append((us * len(dur[k]), name, grid, len(dur[k]), us, rd / 1e6, wr / 1e6, gbs, gbs / (PEAK_HBM / 1e9), busy))
    rows.sort(key=lambda r: -r[0])
    lines = ['| kernel | work-items | calls | median us | read MB | write MB | GB/s | of 8 TB/s | MFMA busy |',
             '|---|---|---|---|---|---|---|---|---|']
    for _, name, grid, n, us, rd, wr, gbs, frac, busy in rows:
        short = name if len(name) < 70 else name[:67] + '...'
        lines.append(f'| `{short}` | {grid} | {n} | {us:.2f} | {rd:.2f} | {wr:.2f} | {gbs:.0f} | {100 * frac:.1f}% | '
                     f'{100 * busy:.1f}% |')
    table = '\n'.join(lines)
    print(table)
    print(json.dumps({'fetch_scale': sf, 'write_scale': sw}))
    return table, sf, sw


def trace_md(trace_csv, title, cmd, desc=None):
    """Markdown summary of a rocprofv3 --kernel-trace CSV: per (kernel, grid) the dispatch
    count and the median / mean duration (the tables under profiles/)."""
    import csv
    import statistics
    by_kg, meta = {}, {}
    for r in csv.DictReader(open(trace_csv)):
        d = (int(r['End_Timestamp']) - int(r['Start_Timestamp'])) / 1e3
        k = (r['Kernel_Name'], (int(r['Grid_Size_X']), int(r['Grid_Size_Y']), int(r['Grid_Size_Z'])))
        by_kg.setdefault(k, []).append(d)
        meta[k] = (r['Workgroup_Size_X'], r['VGPR_Count'], r['Accum_VGPR_Count'], r['LDS_Block_Size'])
    tot = sum(sum(v) for v in by_kg.values())
    out = [f'# {title}', '', 'Command (repo root, one MI355X):', '', '```', cmd, '```', '']
    if desc:
        out += [desc, '']
    out += ['| kernel | grid (work-items x,y,z) | wg | vgpr | agpr | lds B | calls | median us | mean us | time % |',
            '|---|---|---|---|---|---|---|---|---|---|']
    for (k, g), v in sorted(by_kg.items(), key=lambda kv: -sum(kv[1])):
        if sum(v) / tot < 0.002:
            continue
        wg, vg, ag, lds = meta[(k, g)]
        name = k if len(k) < 90 else k[:87] + '...'
        out.append(f'| `{name}` | {g} | {wg} | {vg} | {ag} | {lds} | {len(v)} | {statistics.median(v):.2f} | '
                   f'{statistics.mean(v):.2f} | {100 * sum(v) / tot:.1f} |')
    print('\n'.join(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=20)
    ap.add_argument('--no-ops', action='store_true', help='skip the per-op table of the other configs')
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline')
    ap.add_argument('--per-op-only', action='store_true',
                    help='print only the per-op table (a short program for rocprofv3 kernel traces)')
    ap.add_argument('--traffic-probe', action='store_true', help='short program for the rocprofv3 --pmc passes')
    ap.add_argument('--counters-probe', action='store_true',
                    help='short program for the per-kernel counter table (every forward stage and per-op workload)')
    ap.add_argument('--counters-from', nargs=4, metavar=('TRACE_CSV', 'FETCH_CSV', 'WRITE_CSV', 'SQ_CSV'),
                    help='print the per-kernel counter table from a kernel trace and three --pmc CSVs')
    ap.add_argument('--counters-probe-net', action='store_true',
                    help='short program for the KAD-CNet-S counter table (three eager config-5 forwards)')
    ap.add_argument('--counters-net-from', nargs=4, metavar=('TRACE_CSV', 'FETCH_CSV', 'WRITE_CSV', 'SQ_CSV'),
                    help='print the KAD-CNet-S per-kernel table from a kernel trace and three --pmc CSVs')
    ap.add_argument('--traffic-from', nargs=2, metavar=('FETCH_CSV', 'WRITE_CSV'),
                    help='compute profiles/dsc0_traffic.json from the two --pmc counter CSVs')
    ap.add_argument('--no-kadcnet', action='store_true', help='skip the KAD-CNet-S (config 5) throughput')
    ap.add_argument('--kadcnet-iters', type=int, default=20, help='graph replays per trial for config 5')
    ap.add_argument('--kadcnet-only', action='store_true',
                    help='print only the config-5 throughput (a short program for rocprofv3 kernel traces)')
    ap.add_argument('--trace-md', nargs='+', metavar='ARG',
                    help='TRACE_CSV TITLE COMMAND [DESCRIPTION]: print the markdown summary of a kernel trace')
    args = ap.parse_args()
    if args.trace_md:
        trace_md(*args.trace_md)
        return
    if args.traffic_from:
        traffic_from(*args.traffic_from)
        return
    if args.counters_from:
        counters_from(*args.counters_from)
        return
    if args.counters_net_from:
        counters_net_from(*args.counters_net_from)
        return
    if args.counters_probe_net:
        counters_probe_net()
        return
    if args.counters_probe:
        counters_probe()
        return
    if args.traffic_probe:
        traffic_probe()
        return
    if args.per_op_only:
        with torch.no_grad():
            print(json.dumps(per_op(args.steps, args.warmup, cpu=False)))
        return
    if args.kadcnet_only:
        print(json.dumps(kadcnet_s(args.kadcnet_iters, 5, cpu=False)), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU: every GPU box of this build has one MI355X and the KAD-Conv forward '
              'shards by batch with no exchange; run with --gpus 1', file=sys.stderr)
        sys.exit(2)
    import kadconv
    from kadconv import _ext

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    dtype = torch.float16
    shape = (8, 256, 100, 100)
    m = build_kadconv(256, dtype)
    kadconv.enable_fast_inference(m)
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(0)).to('cuda', dtype)
    with torch.no_grad():
        # whole forward, graph-replayed; bracket with synchronize (one rank: no barrier needed)
        torch.cuda.synchronize()
        us, trials, _ = time_graph(lambda: m(x), args.steps, args.warmup)

        # dominant kernel alone: branch-0 DCN, events on the stream it is launched on
        plan = m._kad_plan
        stages, _ = plan.stages(x)
        for _, fn in stages:
            fn()
        stage_us = {name: round(time_eager(fn, 20), 2) for name, fn in stages}
        sd = dict(stages)
        if 'dsc' in sd:  # grouped: one launch runs every branch's DSC (+ SE)
            dsc0 = sd['dsc']
            flops = sum(dsc_flops(shape[0], shape[2] >> i, shape[3] >> i, br.c) for i, br in enumerate(plan.branches))
            kname = ('dcn_group_kernel<half,half,6,FUSED> (the three branches\' DSCs in one launch: conv_offset + '
                     'DCN + fused SE, c=86/85/85 at 100^2/50^2/25^2, batch 8)')
        else:
            dsc0 = sd['dsc0']
            flops = dsc_flops(shape[0], shape[2], shape[3], plan.branches[0].c)
            kname = 'dcn_fwd_kernel<half,half,6,FUSED> (branch-0 DSC: conv_offset + DCN, c=86, 8x100x100)'
        dcn_us = time_eager(dsc0, args.steps, args.warmup)
        achieved = flops / (dcn_us * 1e-6)

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        traffic = json.load(open(TRAFFIC_FILE)).get('bytes_per_launch')

    out = {
        'metric': 'KAD-Conv fwd us & % roofline at [8,256,100,100] fp16; KAD-CNet-S img/s bs16',
        'value': round(us, 3),
        'unit': 'us',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(us / 1e3, 6),
        'trials_us': [round(t, 3) for t in trials],
        'higher_is_better': False,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f16',
        'data': 'synthetic: x ~ N(0,1) seed 0; weights by state-dict name (seed 0): kaiming-uniform convs, '
                'conv_offset ~ N(0, 2/sqrt(9c)), identity BN, branch scale 1',
        'config': {'workload': 'KADConv(256) forward, x [8,256,100,100] fp16, NCHW, HIP-graph replay',
                   'batch': 8, 'channels': 256, 'hw': [100, 100], 'branches': 3},
        'roofline': {'bound': 'mfma', 'achieved': round(achieved / 1e12, 3), 'peak': PEAK_MFMA_F16 / 1e12,
                     'unit': 'TFLOP/s', 'frac': round(achieved / PEAK_MFMA_F16, 4), 'traffic': traffic,
                     'traffic_source': 'profiles/dsc0_traffic.json (FETCH_SIZE / WRITE_SIZE of bench.py '
                                       '--traffic-probe, scaled by a 64 MiB copy); not measured in this run',
                     'kernel': kname, 'kernel_us': round(dcn_us, 3),
                     'flops_per_launch': flops},
        'forward_roofline': {'floor_us': FORWARD_FLOOR_US, 'frac': round(FORWARD_FLOOR_US / us, 4)},
        'stages_us': stage_us,
        'kadcnet_s_img_per_s': None,
    }
    if not args.no_kadcnet:
        ks = kadcnet_s(args.kadcnet_iters, 5, cpu=not args.no_cpu)
        out['kadcnet_s_img_per_s'] = ks['img_per_s']
        out['kadcnet_s'] = ks
    if not args.no_ops:
        out['per_op'] = per_op(max(args.steps // 4, 20), 5, cpu=not args.no_cpu)
        out['config1'] = config1(max(args.steps // 4, 20), 5, cpu=not args.no_cpu)
    if not args.no_cpu:
        out['cpu_baseline'] = cpu_baseline(shape)
    else:
        out['cpu_baseline'] = None
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
