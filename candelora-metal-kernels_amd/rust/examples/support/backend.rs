// Backend selection (`--backend metal|hip`) for examples/iq2_matmul_bench.rs,
// which includes it with `#[path = "support/backend.rs"] mod backend;`: `Backend::from_arg` parses the
// flag and `Backend::device` creates the device.  With `hip` the device is the
// CPU: the `rocm` bodies of src/iq2_matmul.rs stage the tensors into device
// buffers per call, so the example's latencies include PCIe copies; bench.py
// reports the device-resident throughput of the same C ABI.  Not built here.
use candle_core::{Device, Result};

#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Backend {
    Metal,
    Hip,
}

impl Backend {
    pub fn from_arg(s: &str) -> Result<Self> {
        match s {
            "metal" => Ok(Backend::Metal),
            "hip" => Ok(Backend::Hip),
            other => candle_core::bail!("unknown --backend {other}: expected metal or hip"),
        }
    }

    pub fn device(self) -> Result<Device> {
        match self {
            Backend::Metal => Device::new_metal(0),
            Backend::Hip => {
                if cfg!(feature = "rocm") {
                    Ok(Device::Cpu)
                } else {
                    candle_core::bail!("--backend hip needs a build with --features rocm")
                }
            }
        }
    }

    /// The cargo feature that builds this backend.
    pub fn feature(self) -> &'static str {
        match self {
            Backend::Metal => "metal",
            Backend::Hip => "rocm",
        }
    }
}
