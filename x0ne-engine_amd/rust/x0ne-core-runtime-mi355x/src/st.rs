//! Safetensors files already in memory (x0ne-core/runtime/src/st.rs:216-277, SliceSource): the
//! bytes are handed to the library at Engine::load_from, which checks them (headers, offsets,
//! the index against the files) before any device work.
use std::ffi::CString;

use crate::{Error, Result};

pub struct SliceSource<'a> {
    pub(crate) names: Vec<CString>,
    pub(crate) files: Vec<&'a [u8]>,
    pub(crate) index: Option<CString>,
}

impl<'a> SliceSource<'a> {
    /// `files` are (file name, bytes). Without an index there must be exactly one file.
    pub fn new(index_json: Option<&[u8]>, files: &[(&str, &'a [u8])]) -> Result<Self> {
        if index_json.is_none() && files.len() != 1 {
            return Err(Error::Format(format!("{} files and no index: one file expected", files.len())));
        }
        let names = files
            .iter()
            .map(|(n, _)| CString::new(*n).map_err(|_| Error::Format(format!("file name {n:?} holds a NUL"))))
            .collect::<Result<Vec<_>>>()?;
        let index = match index_json {
            None => None,
            Some(j) => Some(CString::new(j).map_err(|_| Error::Format("index: a NUL byte".into()))?),
        };
        Ok(SliceSource { names, files: files.iter().map(|(_, b)| *b).collect(), index })
    }
}
