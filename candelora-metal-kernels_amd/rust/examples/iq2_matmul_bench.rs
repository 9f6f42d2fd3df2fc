//! IQ2/IQ3 matmul latency bench for either backend of the crate:
//! `cargo run --release --features metal --example iq2_matmul_bench -- --backend metal ...`
//! `cargo run --release --features rocm  --example iq2_matmul_bench -- --backend hip ...`
//!
//! Counterpart of examples/iq2_matmul_bench.rs (same options, same seeded
//! inputs, same output table) with `--backend` added; `support/backend.rs`
//! picks the device (a subfolder, so that cargo does not take it for an
//! example of its own).  Each timed run is one call of
//! `iq2_matmul_with_activation_quant` followed by `device.synchronize()`, timed
//! on the host.  With `hip` the inputs are CPU tensors that the `rocm` body
//! stages to the GPU on every call, so these latencies include the PCIe
//! copies; bench.py reports the device-resident throughput of the same C ABI.
//! Not built in this repository (no Rust toolchain in its image).

#[path = "support/backend.rs"]
mod backend;

use std::time::Instant;

use backend::Backend;
use candelora_metal_kernels::activation_quant::{ActivationQuantConfig, ActivationQuantMode};
use candelora_metal_kernels::iq2_matmul::{iq2_matmul_with_activation_quant, Iq2MatmulVariant};
use candle_core::{DType, Device, Result, Tensor};

const QK: usize = 256;
const ALL_VARIANTS: [(&str, Iq2MatmulVariant); 4] = [
    ("iq2-xxs", Iq2MatmulVariant::Iq2Xxs),
    ("iq2-xs", Iq2MatmulVariant::Iq2Xs),
    ("iq2-s", Iq2MatmulVariant::Iq2S),
    ("iq3-s", Iq2MatmulVariant::Iq3S),
];

struct Options {
    backend: Backend,
    variants: Vec<(&'static str, Iq2MatmulVariant)>,
    mode: ActivationQuantMode,
    m: usize,
    out_dim: usize,
    in_dim: usize,
    warmup_runs: usize,
    runs: usize,
    dtype: DType,
}

const USAGE: &str = "Usage: cargo run --release --features <metal|rocm> --example iq2_matmul_bench -- [options]

Options:
  --backend <metal|hip>  Device backend (default: metal; hip needs --features rocm)
  --variants <csv>       Comma list: iq2-xxs,iq2-xs,iq2-s,iq3-s (default: all four)
  --activation-quant-mode <off|w8a8>
                         Activation quant mode (default: off)
  --m <n>                Batch rows for x (default: 1)
  --out-dim <n>          Output dimension (default: 4096)
  --in-dim <n>           Input dimension (default: 4096)
  --warmup-runs <n>      Warmup runs per variant (default: 5)
  --runs <n>             Measured runs per variant (default: 20)
  --dtype <f16|bf16|f32> Input dtype for x (default: f16)
  --help                 Show this help";

fn bad(msg: String) -> candle_core::Error {
    candle_core::Error::msg(msg)
}

fn count(flag: &str, v: &str) -> Result<usize> {
    v.parse::<usize>().map_err(|e| bad(format!("invalid {flag} `{v}`: {e}")))
}

fn options() -> Result<Options> {
    let mut o = Options {
        backend: Backend::Metal,
        variants: ALL_VARIANTS.to_vec(),
        mode: ActivationQuantMode::Off,
        m: 1,
        out_dim: 4096,
        in_dim: 4096,
        warmup_runs: 5,
        runs: 20,
        dtype: DType::F16,
    };
    let argv: Vec<String> = std::env::args().skip(1).collect();
    let mut i = 0;
    while i < argv.len() {
        let flag = argv[i].as_str();
        if flag == "--help" || flag == "-h" {
            println!("{USAGE}");
            std::process::exit(0);
        }
        let value = argv
            .get(i + 1)
            .ok_or_else(|| bad(format!("missing value for {flag}")))?
            .as_str();
        match flag {
            "--backend" => o.backend = Backend::from_arg(value)?,
            "--variants" => {
                o.variants = value
                    .split(',')
                    .map(str::trim)
                    .filter(|s| !s.is_empty())
                    .map(|s| {
                        ALL_VARIANTS.iter().copied().find(|(name, _)| *name == s).ok_or_else(|| {
                            bad(format!("invalid variant `{s}` (expected iq2-xxs|iq2-xs|iq2-s|iq3-s)"))
                        })
                    })
                    .collect::<Result<Vec<_>>>()?;
                if o.variants.is_empty() {
                    candle_core::bail!("--variants resolved to an empty list");
                }
            }
            "--activation-quant-mode" => {
                o.mode = match value {
                    "off" => ActivationQuantMode::Off,
                    "w8a8" => ActivationQuantMode::W8A8,
                    v => candle_core::bail!("invalid --activation-quant-mode `{v}` (expected off|w8a8)"),
                }
            }
            "--m" => o.m = count(flag, value)?,
            "--out-dim" => o.out_dim = count(flag, value)?,
            "--in-dim" => o.in_dim = count(flag, value)?,
            "--warmup-runs" => o.warmup_runs = count(flag, value)?,
            "--runs" => o.runs = count(flag, value)?,
            "--dtype" => {
                o.dtype = match value {
                    "f16" => DType::F16,
                    "bf16" => DType::BF16,
                    "f32" => DType::F32,
                    v => candle_core::bail!("invalid --dtype `{v}` (expected f16|bf16|f32)"),
                }
            }
            other => candle_core::bail!("unknown option `{other}`"),
        }
        i += 2;
    }
    if o.m == 0 || o.out_dim == 0 || o.in_dim == 0 {
        candle_core::bail!("--m, --out-dim, and --in-dim must all be > 0");
    }
    if o.runs == 0 {
        candle_core::bail!("--runs must be > 0");
    }
    Ok(o)
}

/// Bytes of codes and of scales per 256-weight block (src/iq2_matmul.rs:13-29).
fn block_sizes(v: Iq2MatmulVariant) -> (usize, usize) {
    match v {
        Iq2MatmulVariant::Iq2Xxs => (64, 2),
        Iq2MatmulVariant::Iq2Xs => (64, 10),
        Iq2MatmulVariant::Iq2S => (72, 10),
        Iq2MatmulVariant::Iq3S => (104, 6),
    }
}

/// The crate's seeded bytes: the top byte of each step of the LCG
/// state * 1664525 + 1013904223 (mod 2^32).
fn seeded_bytes(len: usize, seed: u32) -> Vec<u8> {
    std::iter::successors(Some(seed), |s| Some(s.wrapping_mul(1_664_525).wrapping_add(1_013_904_223)))
        .skip(1)
        .take(len)
        .map(|s| (s >> 24) as u8)
        .collect()
}

/// Seeded weights of the bench case: codes and scales from the LCG (seeds
/// xor'ed with the dimensions), every block's d forced to f16 1.0, the last
/// code byte 0x5A.
fn bench_weights(v: Iq2MatmulVariant, out_dim: usize, in_dim: usize) -> (Vec<u8>, Vec<u8>) {
    let blocks = out_dim * in_dim.div_ceil(QK);
    let (bpb, spb) = block_sizes(v);
    let mut codes = seeded_bytes(blocks * bpb, 0xA11C_E5ED ^ out_dim as u32);
    let mut scales = seeded_bytes(blocks * spb, 0xC0FF_EE12 ^ in_dim as u32);
    for block in scales.chunks_exact_mut(spb) {
        block[..2].copy_from_slice(&[0x00, 0x3c]); // f16 1.0, little-endian
    }
    if let Some(b) = codes.last_mut() {
        *b = 0x5A;
    }
    (codes, scales)
}

/// The crate's deterministic activations: ((17 i mod 41) - 20) / 13.
fn bench_x(len: usize) -> Vec<f32> {
    (0..len).map(|i| ((i * 17 % 41) as f32 - 20.0) / 13.0).collect()
}

/// Nearest-rank percentile of sorted values.
fn nearest_rank(sorted: &[f64], p: f64) -> f64 {
    let rank = ((p * sorted.len() as f64).ceil() as usize).max(1);
    sorted[rank.min(sorted.len()) - 1]
}

fn time_variant(device: &Device, o: &Options, v: Iq2MatmulVariant) -> Result<(f64, f64, f64)> {
    let (codes, scales) = bench_weights(v, o.out_dim, o.in_dim);
    let x = Tensor::from_slice(&bench_x(o.m * o.in_dim), (o.m, o.in_dim), device)?.to_dtype(o.dtype)?;
    let codes = Tensor::from_slice(&codes, codes.len(), device)?;
    let scales = Tensor::from_slice(&scales, scales.len(), device)?;
    let quant = ActivationQuantConfig { mode: o.mode, strict: false };
    let call = || -> Result<()> {
        iq2_matmul_with_activation_quant(&x, &codes, &scales, o.out_dim, o.in_dim, v, &quant)?;
        device.synchronize()
    };
    for _ in 0..o.warmup_runs {
        call()?;
    }
    let mut ms = Vec::with_capacity(o.runs);
    for _ in 0..o.runs {
        let t0 = Instant::now();
        call()?;
        ms.push(t0.elapsed().as_secs_f64() * 1e3);
    }
    let mean = ms.iter().sum::<f64>() / ms.len() as f64;
    ms.sort_by(|a, b| a.total_cmp(b));
    Ok((mean, nearest_rank(&ms, 0.50), nearest_rank(&ms, 0.95)))
}

fn main() -> Result<()> {
    let o = options()?;
    let device = o.backend.device()?;
    println!(
        "[iq2-bench] backend={:?} device={:?} dtype={:?} act_quant={:?} shape=({}, {}, {}) warmup_runs={} runs={}",
        o.backend, device, o.dtype, o.mode, o.m, o.out_dim, o.in_dim, o.warmup_runs, o.runs
    );
    println!("[iq2-bench] variants={:?}", o.variants.iter().map(|(n, _)| *n).collect::<Vec<_>>());
    println!("variant\tmean_ms\tp50_ms\tp95_ms\tmatmuls_per_s");
    for &(name, v) in &o.variants {
        let (mean, p50, p95) = time_variant(&device, &o, v)?;
        let rate = if mean > 0.0 { 1e3 / mean } else { 0.0 };
        println!("{name}\t{mean:.3}\t{p50:.3}\t{p95:.3}\t{rate:.3}");
    }
    Ok(())
}
