//! Dynamically loaded host for `libtoktier_hip.so`, the gfx950 (MI355X)
//! tokenizer engine: UTF-8 in, compacted BPE ids out, the whole fresh-encode
//! path on the device.
//!
//! It takes the place of `toktier-cuda-driver` (`crates/toktier-cuda-driver/
//! src/lib.rs:1-642`) on the GPU route. That crate loads the CUDA driver and
//! hands the router contexts, modules, allocations and launches from which
//! `toktier-routing-core/src/gpu.rs` drives the prebuilt kernels itself. Here
//! the library owns the device, the tables, the workspace and the kernel
//! schedule, so this crate exposes an engine: open it with the artifact's
//! tables (the `NativePrebuiltGpu::new` inputs, `gpu.rs:1306-1404`), then
//! encode. The router's `NativeGpuEngine` implementation (`runtime.rs:76-82`)
//! wraps a [`HipEngine`] where it wraps `NativePrebuiltGpu` today.
//!
//! Every function pointer comes from `dlopen`/`dlsym` at [`Library::open`],
//! so a host without the library gets an error, not a link failure. The
//! declarations mirror `include/toktier_hip.h` one for one.

use std::ffi::{c_char, c_int, c_void, CStr, CString};
use std::fmt;
use std::sync::Arc;

pub const TK_ABI_VERSION: u32 = 1;

pub const TK_OK: i32 = 0;
pub const TK_E_INVALID_ARG: i32 = -1;
pub const TK_E_SHAPE: i32 = -2;
pub const TK_E_DEVICE: i32 = -3;
pub const TK_E_ARCH: i32 = -4;
pub const TK_E_UTF8: i32 = -5;
pub const TK_E_NEEDS_NFC: i32 = -6;
pub const TK_E_CAPACITY: i32 = -7;
pub const TK_E_INTERNAL: i32 = -8;
pub const TK_E_UNSUPPORTED: i32 = -9;

pub const TK_FLAG_NORMALIZED: u32 = 1;
pub const TK_FLAG_NO_ADDED: u32 = 2;

pub const TK_ADDED_SPECIAL: u8 = 1;
pub const TK_ADDED_SINGLE_WORD: u8 = 2;
pub const TK_ADDED_LSTRIP: u8 = 4;
pub const TK_ADDED_RSTRIP: u8 = 8;
pub const TK_ADDED_NORMALIZED: u8 = 16;

pub const TK_NOALLOC_MAX_BYTES: usize = 1_048_576;

pub const TK_STAT_LITERALS: usize = 0;
pub const TK_STAT_LONG: usize = 1;
pub const TK_STAT_BIG: usize = 2;
pub const TK_STAT_REPAIRS: usize = 3;

pub const TK_KERNEL_PRETOK: i64 = 0;
pub const TK_KERNEL_BPE_PACK: i64 = 1;
pub const TK_KERNEL_COMPACT: i64 = 2;
pub const TK_KERNEL_BPE_ROWS: i64 = 3;
pub const TK_KERNEL_LONG_WINDOWS: i64 = 4;
pub const TK_KERNEL_ADDED: i64 = 5;
pub const TK_KERNELS: usize = 6;

pub const TK_OPT_COMPACT_PAIRS: c_int = 1;
pub const TK_OPT_REPAIR_WIDEN: c_int = 2;
pub const TK_OPT_TIMED_KERNEL: c_int = 3;
pub const TK_OPT_HOT_PAIRS: c_int = 4;

/// The value of `tk_config.ruleset` for each ruleset.
pub const TK_RULESET_CL100K: i32 = 0;
pub const TK_RULESET_R50K: i32 = 1;
pub const TK_RULESET_LAGUNA: i32 = 2;
pub const TK_RULESET_DEEPSEEK: i32 = 3;
pub const TK_RULESET_O200K: i32 = 4;
pub const TK_RULESET_KIMI: i32 = 5;

/// A failed call: the entry, its `TK_*` status and the library's
/// description (`tk_last_error`).
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct HipError {
    pub call: String,
    pub status: i32,
    pub detail: String,
}

impl HipError {
    fn new(call: &str, status: i32, detail: impl Into<String>) -> Self {
        Self { call: call.to_owned(), status, detail: detail.into() }
    }
}

impl fmt::Display for HipError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "{}: status {}: {}", self.call, self.status, self.detail)
    }
}

impl std::error::Error for HipError {}

/// The kernel families the routing data names (`kernel_families.v1.json`
/// `ruleset`). The strings are the reference's (`gpu.rs:40-62`,
/// `Ruleset::parse`) plus `r50k` (GPT-2), which the reference runs on the
/// CPU only.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Ruleset {
    Cl100k,
    R50k,
    Laguna,
    Deepseek,
    O200k,
    Kimi,
}

impl Ruleset {
    pub fn parse(value: &str) -> Result<Self, HipError> {
        match value {
            "cl100k" => Ok(Self::Cl100k),
            "r50k" => Ok(Self::R50k),
            "laguna" => Ok(Self::Laguna),
            "deepseek" => Ok(Self::Deepseek),
            "o200k" => Ok(Self::O200k),
            "kimi" => Ok(Self::Kimi),
            other => Err(HipError::new(
                "Ruleset::parse",
                TK_E_INVALID_ARG,
                format!("unsupported native GPU ruleset {other:?}"),
            )),
        }
    }

    pub fn as_str(self) -> &'static str {
        match self {
            Self::Cl100k => "cl100k",
            Self::R50k => "r50k",
            Self::Laguna => "laguna",
            Self::Deepseek => "deepseek",
            Self::O200k => "o200k",
            Self::Kimi => "kimi",
        }
    }

    /// `tk_config.ruleset`. The numbering is this library's own and is
    /// never the reference's `Ruleset::numeric()` (cl100k 0, deepseek 1,
    /// laguna 2, none for the windowed group): that value selects kernels
    /// inside the reference's image and does not cross this boundary.
    pub fn code(self) -> i32 {
        match self {
            Self::Cl100k => TK_RULESET_CL100K,
            Self::R50k => TK_RULESET_R50K,
            Self::Laguna => TK_RULESET_LAGUNA,
            Self::Deepseek => TK_RULESET_DEEPSEEK,
            Self::O200k => TK_RULESET_O200K,
            Self::Kimi => TK_RULESET_KIMI,
        }
    }

    /// The class table the ruleset reads (`tk_engine_open`'s
    /// `class_table`), by the routing data's names. Families that keep
    /// combining marks in the letter run (Qwen3.5) take `cl100k_m2l_v3`
    /// with the cl100k ruleset instead.
    pub fn class_table(self) -> &'static str {
        match self {
            Self::Cl100k | Self::R50k | Self::Laguna => "cl100k_v3",
            Self::Deepseek => "deepseek_v1",
            Self::O200k => "o200k_v4",
            Self::Kimi => "kimi_v1",
        }
    }
}

/// What the router knows of an artifact's GPU row; the fields of the
/// reference's `NativePrebuiltGpuConfig` (`gpu.rs:22-38`) that cross this
/// boundary. `ruleset` is the routing data's string.
#[derive(Debug, Clone)]
pub struct HipEngineConfig {
    pub family: String,
    pub artifact_sha256: String,
    /// "gfx950", or empty for any architecture.
    pub expected_architecture: String,
    pub device_ordinal: i32,
    pub ruleset: String,
    pub digits_max: i32,
    pub contractions: bool,
    pub needs_nfc: bool,
    pub ignore_merges: i32,
    pub pair_count: usize,
    pub vocab_count: usize,
}

/// The artifact's tables in the reference's export format
/// (`src/toktier/kernels/bpe_tables.py:1-30`), plus the 0x110000-entry NFC
/// quick-check table for families that normalize.
pub struct Tables<'a> {
    pub class: &'a [u8],
    pub pair_keys: &'a [u64],
    pub pair_vals: &'a [u64],
    pub byte_id: &'a [i32],
    pub vocab_keys: &'a [u64],
    pub vocab_vals: &'a [u64],
    pub vocab_blob: &'a [u8],
    pub unsafe_bits: &'a [u32],
    pub nfc_qc: Option<&'a [u8]>,
}

#[repr(C)]
struct TkConfig {
    abi_version: u32,
    device_ordinal: i32,
    ruleset: i32,
    digits_max: i32,
    contractions: i32,
    needs_nfc: i32,
    ignore_merges: i32,
    pair_count: u64,
    vocab_count: u64,
    family: *const c_char,
    artifact_sha256: *const c_char,
    expected_architecture: *const c_char,
}

#[repr(C)]
struct TkEngine {
    _opaque: [u8; 0],
}

type Preflight = unsafe extern "C" fn(
    *const TkConfig,
    *const u8, usize,
    *const u64, usize,
    *const u64, usize,
    *const i32, usize,
    *const u64, usize,
    *const u64, usize,
    *const u32, usize,
) -> c_int;
type Open = unsafe extern "C" fn(
    *const TkConfig,
    *const u8, usize,
    *const u64, usize,
    *const u64, usize,
    *const i32, usize,
    *const u64, usize,
    *const u64, usize,
    *const u8, usize,
    *const u32, usize,
    *const u8, usize,
    *mut *mut TkEngine,
) -> c_int;
type Close = unsafe extern "C" fn(*mut TkEngine);
type Encode =
    unsafe extern "C" fn(*mut TkEngine, *const u8, usize, u32, *mut u32, usize, *mut usize) -> c_int;
type EncodeBatch = unsafe extern "C" fn(
    *mut TkEngine, *const u8, *const u64, usize, u32, *mut u32, usize, *mut u64, *mut i32,
) -> c_int;
type EncodeBatchDocs = unsafe extern "C" fn(
    *mut TkEngine, *const *const u8, *const usize, usize, u32, *mut u32, usize, *mut u64,
    *mut i32,
) -> c_int;
type EncodeDevice = unsafe extern "C" fn(
    *mut TkEngine, *const c_void, usize, u32, *mut c_void, usize, *mut usize, *mut c_void,
) -> c_int;
type EncodeSeed = unsafe extern "C" fn(
    *mut TkEngine, *const c_void, usize, u32, *mut c_void, usize, u32, *mut c_void, usize,
    *mut usize, *mut usize, *mut c_void,
) -> c_int;
type EncodeSeedHost = unsafe extern "C" fn(
    *mut TkEngine, *const u8, usize, u32, *mut u32, usize, u32, *mut u64, usize, *mut usize,
    *mut usize,
) -> c_int;
type SetAdded = unsafe extern "C" fn(
    *mut TkEngine, usize, *const u8, *const u64, *const u32, *const u8,
) -> c_int;
type LastLiterals = unsafe extern "C" fn(*const TkEngine, *mut u64) -> c_int;
type LastStats = unsafe extern "C" fn(*const TkEngine, *mut u64, c_int) -> c_int;
type DriverVersion = unsafe extern "C" fn(*const TkEngine, *mut c_int) -> c_int;
type Label = unsafe extern "C" fn(*const TkEngine) -> *const c_char;
type SetTiming = unsafe extern "C" fn(*mut TkEngine, c_int) -> c_int;
type LastTiming = unsafe extern "C" fn(*const TkEngine, *mut f64, c_int) -> c_int;
type SetOption = unsafe extern "C" fn(*mut TkEngine, c_int, i64) -> c_int;
type SetFaultMarker = unsafe extern "C" fn(*mut TkEngine, *const u8, usize) -> c_int;
type LastError = unsafe extern "C" fn() -> *const c_char;

struct Api {
    handle: *mut c_void,
    preflight: Preflight,
    open: Open,
    close: Close,
    encode: Encode,
    encode_batch: EncodeBatch,
    encode_batch_docs: EncodeBatchDocs,
    encode_device: EncodeDevice,
    encode_device_noalloc: EncodeDevice,
    encode_seed: EncodeSeed,
    encode_seed_host: EncodeSeedHost,
    set_added: SetAdded,
    last_literals: LastLiterals,
    last_stats: LastStats,
    driver_version: DriverVersion,
    delivery: Label,
    architecture: Label,
    set_timing: SetTiming,
    last_timing: LastTiming,
    set_option: SetOption,
    set_fault_marker: SetFaultMarker,
    last_error: LastError,
}

// The library's entries are thread-safe (each engine serializes its calls;
// tk_last_error is thread-local).
unsafe impl Send for Api {}
unsafe impl Sync for Api {}

impl Drop for Api {
    fn drop(&mut self) {
        unsafe {
            libc::dlclose(self.handle);
        }
    }
}

fn dl_error() -> String {
    unsafe {
        let e = libc::dlerror();
        if e.is_null() {
            "unknown dynamic loader error".to_owned()
        } else {
            CStr::from_ptr(e).to_string_lossy().into_owned()
        }
    }
}

/// One symbol of the library as a function pointer of type `T`.
unsafe fn symbol<T: Copy>(handle: *mut c_void, name: &str) -> Result<T, HipError> {
    let c = CString::new(name).expect("symbol names hold no NUL");
    let p = libc::dlsym(handle, c.as_ptr());
    if p.is_null() {
        return Err(HipError::new("dlsym", TK_E_DEVICE, format!("{name}: {}", dl_error())));
    }
    Ok(std::mem::transmute_copy::<*mut c_void, T>(&p))
}

/// The loaded library. Cheap to clone; engines keep it alive.
#[derive(Clone)]
pub struct Library {
    api: Arc<Api>,
}

impl Library {
    /// Opens the library at `path` (for instance the `toktier_amd/_lib/
    /// libtoktier_hip.so` the build writes, or a bare name the loader
    /// finds on its search path).
    pub fn open(path: &str) -> Result<Self, HipError> {
        let c = CString::new(path)
            .map_err(|_| HipError::new("dlopen", TK_E_INVALID_ARG, "path holds a NUL byte"))?;
        let handle = unsafe { libc::dlopen(c.as_ptr(), libc::RTLD_NOW | libc::RTLD_LOCAL) };
        if handle.is_null() {
            return Err(HipError::new("dlopen", TK_E_DEVICE, format!("{path}: {}", dl_error())));
        }
        let api = unsafe {
            let load = || -> Result<Api, HipError> {
                Ok(Api {
                    handle,
                    preflight: symbol(handle, "tk_engine_preflight")?,
                    open: symbol(handle, "tk_engine_open")?,
                    close: symbol(handle, "tk_engine_close")?,
                    encode: symbol(handle, "tk_engine_encode")?,
                    encode_batch: symbol(handle, "tk_engine_encode_batch")?,
                    encode_batch_docs: symbol(handle, "tk_engine_encode_batch_docs")?,
                    encode_device: symbol(handle, "tk_engine_encode_device")?,
                    encode_device_noalloc: symbol(handle, "tk_engine_encode_device_noalloc")?,
                    encode_seed: symbol(handle, "tk_engine_encode_seed")?,
                    encode_seed_host: symbol(handle, "tk_engine_encode_seed_host")?,
                    set_added: symbol(handle, "tk_engine_set_added")?,
                    last_literals: symbol(handle, "tk_engine_last_literals")?,
                    last_stats: symbol(handle, "tk_engine_last_stats")?,
                    driver_version: symbol(handle, "tk_engine_driver_version")?,
                    delivery: symbol(handle, "tk_engine_delivery")?,
                    architecture: symbol(handle, "tk_engine_architecture")?,
                    set_timing: symbol(handle, "tk_engine_set_timing")?,
                    last_timing: symbol(handle, "tk_engine_last_timing")?,
                    set_option: symbol(handle, "tk_engine_set_option")?,
                    set_fault_marker: symbol(handle, "tk_engine_set_fault_marker")?,
                    last_error: symbol(handle, "tk_last_error")?,
                })
            };
            match load() {
                Ok(api) => api,
                Err(e) => {
                    libc::dlclose(handle);
                    return Err(e);
                }
            }
        };
        Ok(Self { api: Arc::new(api) })
    }

    fn check(&self, call: &str, status: c_int) -> Result<(), HipError> {
        if status == TK_OK {
            return Ok(());
        }
        let detail = unsafe {
            let p = (self.api.last_error)();
            if p.is_null() {
                String::new()
            } else {
                CStr::from_ptr(p).to_string_lossy().into_owned()
            }
        };
        Err(HipError::new(call, status, detail))
    }

    /// The device-free shape checks of `tk_engine_open` (the reference's
    /// `NativePrebuiltGpu::preflight`, `gpu.rs:1383-1404`, and the shape
    /// rules of `validate_tables`, `gpu.rs:1642-1679`).
    pub fn preflight(&self, cfg: &HipEngineConfig, t: &Tables<'_>) -> Result<(), HipError> {
        let owned = OwnedConfig::new(cfg)?;
        let st = unsafe {
            (self.api.preflight)(
                &owned.raw,
                t.class.as_ptr(), bytes(t.class),
                t.pair_keys.as_ptr(), bytes(t.pair_keys),
                t.pair_vals.as_ptr(), bytes(t.pair_vals),
                t.byte_id.as_ptr(), bytes(t.byte_id),
                t.vocab_keys.as_ptr(), bytes(t.vocab_keys),
                t.vocab_vals.as_ptr(), bytes(t.vocab_vals),
                t.unsafe_bits.as_ptr(), bytes(t.unsafe_bits),
            )
        };
        self.check("tk_engine_preflight", st)
    }

    /// Opens the device named by `cfg.device_ordinal` and uploads the
    /// tables (`NativePrebuiltGpu::new`).
    pub fn open_engine(&self, cfg: &HipEngineConfig, t: &Tables<'_>) -> Result<HipEngine, HipError> {
        let owned = OwnedConfig::new(cfg)?;
        let nfc = t.nfc_qc.unwrap_or(&[]);
        let mut raw: *mut TkEngine = std::ptr::null_mut();
        let st = unsafe {
            (self.api.open)(
                &owned.raw,
                t.class.as_ptr(), bytes(t.class),
                t.pair_keys.as_ptr(), bytes(t.pair_keys),
                t.pair_vals.as_ptr(), bytes(t.pair_vals),
                t.byte_id.as_ptr(), bytes(t.byte_id),
                t.vocab_keys.as_ptr(), bytes(t.vocab_keys),
                t.vocab_vals.as_ptr(), bytes(t.vocab_vals),
                t.vocab_blob.as_ptr(), bytes(t.vocab_blob),
                t.unsafe_bits.as_ptr(), bytes(t.unsafe_bits),
                if nfc.is_empty() { std::ptr::null() } else { nfc.as_ptr() }, nfc.len(),
                &mut raw,
            )
        };
        self.check("tk_engine_open", st)?;
        Ok(HipEngine { lib: self.clone(), raw })
    }
}

fn bytes<T>(s: &[T]) -> usize {
    std::mem::size_of_val(s)
}

/// A `TkConfig` with the C strings it points to.
struct OwnedConfig {
    raw: TkConfig,
    _strings: [CString; 3],
}

impl OwnedConfig {
    fn new(cfg: &HipEngineConfig) -> Result<Self, HipError> {
        let ruleset = Ruleset::parse(&cfg.ruleset)?;
        let cstr = |s: &str| {
            CString::new(s).map_err(|_| {
                HipError::new("tk_config", TK_E_INVALID_ARG, "a label holds a NUL byte")
            })
        };
        let strings = [
            cstr(&cfg.family)?,
            cstr(&cfg.artifact_sha256)?,
            cstr(&cfg.expected_architecture)?,
        ];
        let raw = TkConfig {
            abi_version: TK_ABI_VERSION,
            device_ordinal: cfg.device_ordinal,
            ruleset: ruleset.code(),
            digits_max: cfg.digits_max,
            contractions: cfg.contractions as i32,
            needs_nfc: cfg.needs_nfc as i32,
            ignore_merges: cfg.ignore_merges,
            pair_count: cfg.pair_count as u64,
            vocab_count: cfg.vocab_count as u64,
            family: strings[0].as_ptr(),
            artifact_sha256: strings[1].as_ptr(),
            expected_architecture: if cfg.expected_architecture.is_empty() {
                std::ptr::null()
            } else {
                strings[2].as_ptr()
            },
        };
        Ok(Self { raw, _strings: strings })
    }
}

/// Rows of a batch: per document its ids, or its own error (for instance
/// `TK_E_NEEDS_NFC`, which the caller resolves by normalizing that
/// document and encoding it again with `TK_FLAG_NORMALIZED`).
pub type BatchRows = Vec<Result<Vec<u32>, HipError>>;

/// An open engine on one device. The library serializes the calls on one
/// engine, so it is shared across threads as is.
pub struct HipEngine {
    lib: Library,
    raw: *mut TkEngine,
}

unsafe impl Send for HipEngine {}
unsafe impl Sync for HipEngine {}

impl Drop for HipEngine {
    fn drop(&mut self) {
        unsafe { (self.lib.api.close)(self.raw) }
    }
}

impl HipEngine {
    fn check(&self, call: &str, status: c_int) -> Result<(), HipError> {
        self.lib.check(call, status)
    }

    /// One request, host buffers (`NativeGpuEngine::encode_ids`). A text
    /// that fails the NFC quick check returns `TK_E_NEEDS_NFC`.
    pub fn encode(&self, text: &[u8], flags: u32) -> Result<Vec<u32>, HipError> {
        let mut ids = vec![0u32; text.len().max(1)];
        let mut n = 0usize;
        let st = unsafe {
            (self.lib.api.encode)(self.raw, text.as_ptr(), text.len(), flags, ids.as_mut_ptr(),
                                  ids.len(), &mut n)
        };
        self.check("tk_engine_encode", st)?;
        ids.truncate(n);
        Ok(ids)
    }

    /// A batch in one device pass (`NativeGpuEngine::encode_batch_ids`);
    /// each row equals [`encode`](Self::encode) of that document alone. A
    /// failure of the whole call is every row's error. The documents stay
    /// where they are: the engine's copy threads gather them into its
    /// pinned staging (`tk_engine_encode_batch_docs`).
    pub fn encode_batch(&self, docs: &[&[u8]], flags: u32) -> BatchRows {
        let ptrs: Vec<*const u8> = docs.iter().map(|d| d.as_ptr()).collect();
        let lens: Vec<usize> = docs.iter().map(|d| d.len()).collect();
        let total: usize = lens.iter().sum();
        let mut ids = vec![0u32; total.max(1)];
        let mut rows = vec![0u64; docs.len() + 1];
        let mut status = vec![0i32; docs.len().max(1)];
        let st = unsafe {
            (self.lib.api.encode_batch_docs)(self.raw, ptrs.as_ptr(), lens.as_ptr(), docs.len(),
                                             flags, ids.as_mut_ptr(), ids.len(),
                                             rows.as_mut_ptr(), status.as_mut_ptr())
        };
        if let Err(e) = self.check("tk_engine_encode_batch_docs", st) {
            return docs.iter().map(|_| Err(e.clone())).collect();
        }
        (0..docs.len())
            .map(|d| match status[d] {
                TK_OK => Ok(ids[rows[d] as usize..rows[d + 1] as usize].to_vec()),
                s => Err(HipError::new("tk_engine_encode_batch_docs row", s,
                                       format!("document {d}"))),
            })
            .collect()
    }

    /// Device-resident form: `d_text` and `d_ids` are device addresses on
    /// the engine's device, `stream` a `hipStream_t` or null for the
    /// engine's own. Returns the id count.
    ///
    /// # Safety
    /// The addresses must hold `nbytes` and `ids_cap` entries.
    pub unsafe fn encode_device(&self, d_text: *const c_void, nbytes: usize, flags: u32,
                                d_ids: *mut c_void, ids_cap: usize, stream: *mut c_void)
                                -> Result<usize, HipError> {
        let mut n = 0usize;
        let st = (self.lib.api.encode_device)(self.raw, d_text, nbytes, flags, d_ids, ids_cap,
                                              &mut n, stream);
        self.check("tk_engine_encode_device", st)?;
        Ok(n)
    }

    /// [`encode_device`](Self::encode_device) without any device
    /// allocation (the library's static scratch array), for inputs of at
    /// most `TK_NOALLOC_MAX_BYTES`; not for a stream under graph capture.
    ///
    /// # Safety
    /// As for `encode_device`.
    pub unsafe fn encode_device_noalloc(&self, d_text: *const c_void, nbytes: usize, flags: u32,
                                        d_ids: *mut c_void, ids_cap: usize,
                                        stream: *mut c_void) -> Result<usize, HipError> {
        let mut n = 0usize;
        let st = (self.lib.api.encode_device_noalloc)(self.raw, d_text, nbytes, flags, d_ids,
                                                      ids_cap, &mut n, stream);
        self.check("tk_engine_encode_device_noalloc", st)?;
        Ok(n)
    }

    /// The session seed with device buffers: ids plus, for every token
    /// index `k * stride`, three u64 at `d_points` (the store's
    /// `SpanCheckpoint`, `toktier-store-core/src/tail.rs:17-31`). Returns
    /// (ids, checkpoints).
    ///
    /// # Safety
    /// The addresses must hold `nbytes`, `ids_cap` and `3 * points_cap`
    /// entries.
    pub unsafe fn encode_seed(&self, d_text: *const c_void, nbytes: usize, flags: u32,
                              d_ids: *mut c_void, ids_cap: usize, stride: u32,
                              d_points: *mut c_void, points_cap: usize, stream: *mut c_void)
                              -> Result<(usize, usize), HipError> {
        let (mut n, mut m) = (0usize, 0usize);
        let st = (self.lib.api.encode_seed)(self.raw, d_text, nbytes, flags, d_ids, ids_cap,
                                            stride, d_points, points_cap, &mut n, &mut m, stream);
        self.check("tk_engine_encode_seed", st)?;
        Ok((n, m))
    }

    /// The session seed with host buffers: the ids and the checkpoints
    /// (`[first byte, first byte of its character, character index]` per
    /// `stride` tokens).
    pub fn encode_seed_host(&self, text: &[u8], flags: u32, stride: u32)
                            -> Result<(Vec<u32>, Vec<[u64; 3]>), HipError> {
        let mut ids = vec![0u32; text.len().max(1)];
        let stride_n = stride.max(1) as usize;
        let points_cap = ids.len().div_ceil(stride_n);
        let mut points = vec![0u64; 3 * points_cap.max(1)];
        let (mut n, mut m) = (0usize, 0usize);
        let st = unsafe {
            (self.lib.api.encode_seed_host)(self.raw, text.as_ptr(), text.len(), flags,
                                            ids.as_mut_ptr(), ids.len(), stride,
                                            points.as_mut_ptr(), points_cap, &mut n, &mut m)
        };
        self.check("tk_engine_encode_seed_host", st)?;
        ids.truncate(n);
        let cps = points[..3 * m].chunks_exact(3).map(|c| [c[0], c[1], c[2]]).collect();
        Ok((ids, cps))
    }

    /// The artifact's added tokens, in artifact order: (content, id,
    /// `TK_ADDED_*` flags). An empty slice removes the table.
    pub fn set_added(&self, added: &[(&str, u32, u8)]) -> Result<(), HipError> {
        let mut contents = Vec::new();
        let mut offsets = Vec::with_capacity(added.len() + 1);
        let mut ids = Vec::with_capacity(added.len());
        let mut flags = Vec::with_capacity(added.len());
        offsets.push(0u64);
        for (c, id, f) in added {
            contents.extend_from_slice(c.as_bytes());
            offsets.push(contents.len() as u64);
            ids.push(*id);
            flags.push(*f);
        }
        let st = unsafe {
            (self.lib.api.set_added)(self.raw, added.len(), contents.as_ptr(), offsets.as_ptr(),
                                     ids.as_ptr(), flags.as_ptr())
        };
        self.check("tk_engine_set_added", st)
    }

    /// Literals the last encode extracted (the `R_INPUT_ADDED_TOKEN`
    /// ledger fact, `runtime.rs:648-654`).
    pub fn last_literals(&self) -> Result<u64, HipError> {
        let mut n = 0u64;
        let st = unsafe { (self.lib.api.last_literals)(self.raw, &mut n) };
        self.check("tk_engine_last_literals", st)?;
        Ok(n)
    }

    /// `[literals, pieces over 64 B, pieces over 512 B, repair passes]` of
    /// the last encode (`TK_STAT_*`).
    pub fn last_stats(&self) -> Result<[u64; 4], HipError> {
        let mut out = [0u64; 4];
        let st = unsafe { (self.lib.api.last_stats)(self.raw, out.as_mut_ptr(), 4) };
        if st < 0 {
            self.check("tk_engine_last_stats", st)?;
        }
        Ok(out)
    }

    /// HIP driver version of the engine's device, for the route's driver
    /// floor (`CudaContext::driver_version`).
    pub fn driver_version(&self) -> Result<i32, HipError> {
        let mut v: c_int = 0;
        let st = unsafe { (self.lib.api.driver_version)(self.raw, &mut v) };
        self.check("tk_engine_driver_version", st)?;
        Ok(v)
    }

    /// The audited delivery label the route reports ("prebuilt").
    pub fn delivery(&self) -> String {
        label(unsafe { (self.lib.api.delivery)(self.raw) })
    }

    /// The device's architecture ("gfx950").
    pub fn architecture(&self) -> String {
        label(unsafe { (self.lib.api.architecture)(self.raw) })
    }

    /// Timing mode: 0 off, 1 every stage and kernel, 2 one kernel
    /// (`TK_OPT_TIMED_KERNEL`).
    pub fn set_timing(&self, mode: i32) -> Result<(), HipError> {
        let st = unsafe { (self.lib.api.set_timing)(self.raw, mode) };
        self.check("tk_engine_set_timing", st)
    }

    /// Microsecond times of the last encode (`8 + TK_KERNELS` values).
    pub fn last_timing(&self) -> Result<Vec<f64>, HipError> {
        let mut us = vec![0f64; 8 + TK_KERNELS];
        let st = unsafe { (self.lib.api.last_timing)(self.raw, us.as_mut_ptr(), us.len() as c_int) };
        if st < 0 {
            self.check("tk_engine_last_timing", st)?;
        }
        us.truncate(st.max(0) as usize);
        Ok(us)
    }

    /// `TK_OPT_*` engine options.
    pub fn set_option(&self, option: c_int, value: i64) -> Result<(), HipError> {
        let st = unsafe { (self.lib.api.set_option)(self.raw, option, value) };
        self.check("tk_engine_set_option", st)
    }

    /// Test-only fault injection (the stand-in for the reference's
    /// `PoisonEncoder`, `gpu.rs:1828-1854`); an empty marker clears it.
    pub fn set_fault_marker(&self, marker: &[u8]) -> Result<(), HipError> {
        let st = unsafe {
            (self.lib.api.set_fault_marker)(self.raw, marker.as_ptr(), marker.len())
        };
        self.check("tk_engine_set_fault_marker", st)
    }
}

fn label(p: *const c_char) -> String {
    if p.is_null() {
        String::new()
    } else {
        unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
    }
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn ruleset_strings_round_trip() {
        for s in ["cl100k", "r50k", "laguna", "deepseek", "o200k", "kimi"] {
            assert_eq!(Ruleset::parse(s).unwrap().as_str(), s);
        }
        assert!(Ruleset::parse("cl100k_base").is_err());
    }

    #[test]
    fn ruleset_codes_are_the_headers() {
        assert_eq!(Ruleset::parse("cl100k").unwrap().code(), 0);
        assert_eq!(Ruleset::parse("deepseek").unwrap().code(), 3);
        assert_eq!(Ruleset::parse("laguna").unwrap().code(), 2);
        assert_eq!(Ruleset::parse("o200k").unwrap().code(), 4);
        assert_eq!(Ruleset::parse("kimi").unwrap().code(), 5);
    }

    #[test]
    fn config_layout_matches_the_header() {
        // seven 32-bit fields, padding to 8, two u64, three pointers
        assert_eq!(std::mem::size_of::<TkConfig>(), 32 + 16 + 3 * std::mem::size_of::<usize>());
    }
}
